// Element-level operators of the reference's public API on the device:
// bit packing of base codes, 4-bit residual slots, the fp32 quantizer path
// and the single-page base write.
//
// Reference semantics (paths relative to the reference root):
//   pack_int{2,3,4}[_2d], unpack_*, pack_codes_2d   quantizer.py:147-383
//   quantize / dequantize (fp32 arithmetic)        quantizer.py:31-82
//   pack_4bit / unpack_4bit                        residual_store.py:121-146
//   CAREKVCache.write_base                         cache.py:592-654
#include "common.h"
#include "host_util.h"

namespace carekv {

// Codes per packing unit and bytes per unit: INT3 packs 8 codes into a
// 24-bit little-endian word (3 bytes), INT2 4 codes and INT4 2 codes into one
// byte, LSB first (quantizer.py:147-324).
__host__ __device__ constexpr int unit_codes(int bits) { return bits == 3 ? 8 : 8 / bits; }
__host__ __device__ constexpr int unit_bytes(int bits) { return bits == 3 ? 3 : 1; }

template <int BITS>
__global__ void pack_codes_kernel(const int8_t* __restrict__ codes, long units, int8_t* __restrict__ packed) {
  constexpr int NC = unit_codes(BITS), NB = unit_bytes(BITS);
  const long u = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < NC; ++i) w |= ((uint32_t)(uint8_t)codes[u * NC + i] & ((1u << BITS) - 1u)) << (BITS * i);
#pragma unroll
  for (int b = 0; b < NB; ++b) packed[u * NB + b] = (int8_t)(uint8_t)(w >> (8 * b));
}

template <int BITS>
__global__ void unpack_codes_kernel(const int8_t* __restrict__ packed, long units, int8_t* __restrict__ codes) {
  constexpr int NC = unit_codes(BITS), NB = unit_bytes(BITS);
  const long u = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  uint32_t w = 0;
#pragma unroll
  for (int b = 0; b < NB; ++b) w |= (uint32_t)(uint8_t)packed[u * NB + b] << (8 * b);
  constexpr int half_range = 1 << (BITS - 1);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int v = (int)((w >> (BITS * i)) & ((1u << BITS) - 1u));
    codes[u * NC + i] = (int8_t)(v >= half_range ? v - 2 * half_range : v);  // sign extension
  }
}

// pack_4bit over the whole input in one work-group: s = max|x| / 7 (clamped
// at 1e-8 in the input's dtype), codes clamp(round(x / s), -8, 7) in the
// input's arithmetic, pairs lo | hi << 4, stored scale half(s).
template <bool F16IN>
__global__ __launch_bounds__(1024) void pack_4bit_kernel(const void* __restrict__ xv, long numel,
                                                         int8_t* __restrict__ packed, uint16_t* __restrict__ scale) {
  __shared__ float red[16];
  const float* xf = (const float*)xv;
  const uint16_t* xh = (const uint16_t*)xv;
  auto ld = [&](long i) { return F16IN ? h2f(xh[i]) : xf[i]; };
  float m = 0.f;
  for (long i = threadIdx.x; i < numel; i += blockDim.x) m = fmaxf(m, fabsf(ld(i)));
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x < 64) {
    float v = threadIdx.x < (blockDim.x >> 6) ? red[threadIdx.x] : 0.f;
    v = wave_max(v);
    if (threadIdx.x == 0) red[0] = v;
  }
  __syncthreads();
  m = red[0];
  float s;
  if constexpr (F16IN) {
    s = (float)(_Float16)(m / 7.f);  // the fp16 clamp at 1e-8 is 0
  } else {
    s = fmaxf(m, 1e-8f) / 7.f;
  }
  if (threadIdx.x == 0) scale[0] = f2h(s);
  auto code = [&](long i) -> uint32_t {
    if (i >= numel) return 0u;
    float q = F16IN ? (float)(_Float16)(ld(i) / s) : ld(i) / s;
    q = fminf(fmaxf(rintf(q), -8.f), 7.f);
    return (uint32_t)((int)q) & 15u;
  };
  for (long p = threadIdx.x; p < (numel + 1) / 2; p += blockDim.x)
    packed[p] = (int8_t)(uint8_t)(code(2 * p) | (code(2 * p + 1) << 4));
}

__global__ void unpack_4bit_kernel(const int8_t* __restrict__ packed, const uint16_t* __restrict__ scale, long numel,
                                   float* __restrict__ out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= numel) return;
  const uint32_t b = (uint8_t)packed[i >> 1];
  const int v = (int)((i & 1) ? (b >> 4) : (b & 15u));
  out[i] = (float)(v > 7 ? v - 16 : v) * h2f(scale[0]);
}

// fp32 quantizer (quantizer.py:42-64 with an fp32 input): max|x| clamped at
// 1e-8, scale = max / qmax, code = clamp(round(x / scale)).  One thread per
// group of 32.
template <int BITS>
__global__ void quantize_rows_f32_kernel(const float* __restrict__ x, long groups, int8_t* __restrict__ codes,
                                         float* __restrict__ scale) {
  constexpr int qmax = (1 << (BITS - 1)) - 1;
  const long gi = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const float* xp = x + gi * 32;
  float m = 0.f;
  for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(xp[i]));
  const float s = fmaxf(m, 1e-8f) / (float)qmax;
  scale[gi] = s;
  for (int i = 0; i < 32; ++i) {
    const float q = fminf(fmaxf(rintf(xp[i] / s), (float)(-qmax - 1)), (float)qmax);
    codes[gi * 32 + i] = (int8_t)(int)q;
  }
}

__global__ void dequantize_rows_f32_kernel(const int8_t* __restrict__ codes, const float* __restrict__ scale, long n,
                                           float* __restrict__ out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (float)codes[i] * scale[i / 32];
}

// write_base of one page (cache.py:617-654): pack the page's 16 code rows,
// encode its scales (int8 codes under a per-page fp16 master over the
// page's 16 x G scales, cache.py:592-604, or the fp16 scales), set valid.
// One wave; lane l = row l / NG, group l % NG.
template <int D, int BITS>
__global__ __launch_bounds__(64) void write_base_kernel(carekv_arena A, long pg, const int8_t* __restrict__ kc,
                                                        const uint16_t* __restrict__ ks,
                                                        const int8_t* __restrict__ vc,
                                                        const uint16_t* __restrict__ vs, int num_valid) {
  constexpr int NG = D / 32, RB = row_bytes(D, BITS), CB = 4 * BITS;
  const int lane = threadIdx.x;
  const int r = lane / NG, g = lane % NG;
  const bool cell = lane < kPage * NG;
  float sk = 0.f, sv = 0.f;
  if (cell) {
#pragma unroll
    for (int which = 0; which < 2; ++which) {
      const int8_t* c = (which ? vc : kc) + (long)r * D + g * 32;
      uint32_t w[BITS];
#pragma unroll
      for (int i = 0; i < BITS; ++i) w[i] = 0;
      for (int k = 0; k < 32; ++k) {
        const uint32_t u = (uint32_t)(uint8_t)c[k] & ((1u << BITS) - 1u);
        const int bit = BITS * k;
        w[bit >> 5] |= u << (bit & 31);
        if ((bit & 31) + BITS > 32) w[(bit >> 5) + 1] |= u >> (32 - (bit & 31));
      }
      store_bytes<CB>((which ? A.vcodes : A.kcodes) + (pg * kPage + r) * RB + g * CB, w);
    }
    sk = h2f(ks[r * NG + g]);
    sv = h2f(vs[r * NG + g]);
  }
  if (A.scale_mode == 1) {
    const float mk = (float)(_Float16)(wave_max(cell ? fabsf(sk) : 0.f) / 127.f);
    const float mv = (float)(_Float16)(wave_max(cell ? fabsf(sv) : 0.f) / 127.f);
    auto code = [](float s, float m) -> int8_t {
      const float q = s / m;
      if (q != q) return 0;
      return (int8_t)fminf(fmaxf(rintf(q), -128.f), 127.f);
    };
    if (cell) {
      ((int8_t*)A.kscale)[(pg * kPage + r) * NG + g] = code(sk, mk);
      ((int8_t*)A.vscale)[(pg * kPage + r) * NG + g] = code(sv, mv);
    }
    if (lane == 0) { A.kmaster[pg] = f2h(mk); A.vmaster[pg] = f2h(mv); }
  } else if (cell) {
    ((uint16_t*)A.kscale)[(pg * kPage + r) * NG + g] = ks[r * NG + g];
    ((uint16_t*)A.vscale)[(pg * kPage + r) * NG + g] = vs[r * NG + g];
  }
  if (lane == 0) A.valid[pg] = num_valid;
}

}  // namespace carekv

using namespace carekv;

namespace {
unsigned blocks_of(long n, int per) { return (unsigned)((n + per - 1) / per); }
}  // namespace

extern "C" int carekv_pack_codes(const int8_t* codes, int64_t rows, int32_t D, int32_t bits, int8_t* packed,
                                 void* stream) {
  CAREKV_REQUIRE(codes && packed, "null argument");
  CAREKV_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3 or 4");
  CAREKV_REQUIRE(D > 0 && D % unit_codes(bits) == 0, "D must be a multiple of 8 (INT3), 4 (INT2) or 2 (INT4)");
  CAREKV_REQUIRE(rows >= 0, "negative rows");
  const long units = rows * (long)(D / unit_codes(bits));
  if (units == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(blocks_of(units, 256));
  if (bits == 2) hipLaunchKernelGGL(pack_codes_kernel<2>, grid, dim3(256), 0, s, codes, units, packed);
  else if (bits == 3) hipLaunchKernelGGL(pack_codes_kernel<3>, grid, dim3(256), 0, s, codes, units, packed);
  else hipLaunchKernelGGL(pack_codes_kernel<4>, grid, dim3(256), 0, s, codes, units, packed);
  CAREKV_CHECK_LAUNCH("pack_codes");
  return CAREKV_OK;
}

extern "C" int carekv_unpack_codes(const int8_t* packed, int64_t rows, int32_t D, int32_t bits, int8_t* codes,
                                   void* stream) {
  CAREKV_REQUIRE(codes && packed, "null argument");
  CAREKV_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3 or 4");
  CAREKV_REQUIRE(D > 0 && D % unit_codes(bits) == 0, "D must be a multiple of 8 (INT3), 4 (INT2) or 2 (INT4)");
  CAREKV_REQUIRE(rows >= 0, "negative rows");
  const long units = rows * (long)(D / unit_codes(bits));
  if (units == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(blocks_of(units, 256));
  if (bits == 2) hipLaunchKernelGGL(unpack_codes_kernel<2>, grid, dim3(256), 0, s, packed, units, codes);
  else if (bits == 3) hipLaunchKernelGGL(unpack_codes_kernel<3>, grid, dim3(256), 0, s, packed, units, codes);
  else hipLaunchKernelGGL(unpack_codes_kernel<4>, grid, dim3(256), 0, s, packed, units, codes);
  CAREKV_CHECK_LAUNCH("unpack_codes");
  return CAREKV_OK;
}

extern "C" int carekv_pack_4bit(const void* x, int32_t x_fp16, int64_t numel, int8_t* packed, uint16_t* scale,
                                void* stream) {
  CAREKV_REQUIRE(x && packed && scale, "null argument");
  CAREKV_REQUIRE(numel > 0, "numel must be positive");
  hipStream_t s = (hipStream_t)stream;
  if (x_fp16) hipLaunchKernelGGL(pack_4bit_kernel<true>, dim3(1), dim3(1024), 0, s, x, (long)numel, packed, scale);
  else hipLaunchKernelGGL(pack_4bit_kernel<false>, dim3(1), dim3(1024), 0, s, x, (long)numel, packed, scale);
  CAREKV_CHECK_LAUNCH("pack_4bit");
  return CAREKV_OK;
}

extern "C" int carekv_unpack_4bit(const int8_t* packed, const uint16_t* scale, int64_t numel, float* out,
                                  void* stream) {
  CAREKV_REQUIRE(packed && scale && out, "null argument");
  if (numel <= 0) return CAREKV_OK;
  hipLaunchKernelGGL(unpack_4bit_kernel, dim3(blocks_of(numel, 256)), dim3(256), 0, (hipStream_t)stream, packed, scale,
                     (long)numel, out);
  CAREKV_CHECK_LAUNCH("unpack_4bit");
  return CAREKV_OK;
}

extern "C" int carekv_quantize_rows_f32(const float* x, int64_t rows, int32_t D, int32_t bits, int32_t group,
                                        int8_t* codes, float* scale, void* stream) {
  CAREKV_REQUIRE(x && codes && scale, "null argument");
  CAREKV_REQUIRE(group == 32 && D % 32 == 0 && D > 0, "kernels support group_size=32 and D % 32 == 0");
  CAREKV_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3 or 4");
  const long groups = rows * (long)(D / 32);
  if (groups <= 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(blocks_of(groups, 256));
  if (bits == 2) hipLaunchKernelGGL(quantize_rows_f32_kernel<2>, grid, dim3(256), 0, s, x, groups, codes, scale);
  else if (bits == 3) hipLaunchKernelGGL(quantize_rows_f32_kernel<3>, grid, dim3(256), 0, s, x, groups, codes, scale);
  else hipLaunchKernelGGL(quantize_rows_f32_kernel<4>, grid, dim3(256), 0, s, x, groups, codes, scale);
  CAREKV_CHECK_LAUNCH("quantize_rows_f32");
  return CAREKV_OK;
}

extern "C" int carekv_dequantize_rows_f32(const int8_t* codes, const float* scale, int64_t rows, int32_t D,
                                          int32_t group, float* out, void* stream) {
  CAREKV_REQUIRE(codes && scale && out, "null argument");
  CAREKV_REQUIRE(group == 32 && D % 32 == 0 && D > 0, "kernels support group_size=32 and D % 32 == 0");
  const long n = rows * (long)D;
  if (n <= 0) return CAREKV_OK;
  hipLaunchKernelGGL(dequantize_rows_f32_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, (hipStream_t)stream, codes,
                     scale, n, out);
  CAREKV_CHECK_LAUNCH("dequantize_rows_f32");
  return CAREKV_OK;
}

extern "C" int carekv_write_base(const carekv_arena* arena, int32_t seq, int32_t kv_head, int32_t page,
                                 const int8_t* k_codes, const uint16_t* k_scale, const int8_t* v_codes,
                                 const uint16_t* v_scale, int32_t num_valid, void* stream) {
  CAREKV_REQUIRE(arena && k_codes && k_scale && v_codes && v_scale, "null argument");
  const carekv_arena& A = *arena;
  CAREKV_REQUIRE(check_arena(A), last_error_buf());
  CAREKV_REQUIRE(A.base_bits != 16, "the fp16 side-buffer base is written with write_base_kivi");
  CAREKV_REQUIRE(seq >= 0 && seq < A.n_seq && kv_head >= 0 && kv_head < A.n_kv_heads, "seq / kv_head out of range");
  CAREKV_REQUIRE(page >= 0 && page < A.max_pages, "page out of range");
  CAREKV_REQUIRE(num_valid >= 0 && num_valid <= kPage, "num_valid must be in 0..page_size");
  const long pg = ((long)kv_head * A.n_seq + seq) * A.max_pages + page;
  hipStream_t s = (hipStream_t)stream;
  return dispatch_db(A.head_dim, A.base_bits, [&](auto d, auto b) {
    hipLaunchKernelGGL((write_base_kernel<decltype(d)::value, decltype(b)::value>), dim3(1), dim3(64), 0, s, A, pg,
                       k_codes, k_scale, v_codes, v_scale, (int)num_valid);
    CAREKV_CHECK_LAUNCH("write_base");
    return CAREKV_OK;
  });
}
