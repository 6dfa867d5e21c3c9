// Work-group (256 threads, 4 waves) reductions and scans with a fixed
// combination order, so results do not depend on scheduling.
#pragma once

#include "common.h"

namespace carekv {

constexpr int kBlock = 256;

// Work-group scratch of the reductions below: wave totals and broadcast
// slots (small, so that it costs little of a work-group's LDS).
struct BlockScratch {
  float f[16];
  int i[16];
  int wsum[4];
  int bc[8];
};

// Butterfly wave reductions (fixed pattern: every lane ends with the same
// bits).
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Four sums over the block with one barrier pair: wave butterflies, then
// the 4 wave totals in wave order.
__device__ __forceinline__ void block_sum4(float& a, float& b, int& c, int& d, BlockScratch& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  a = wave_sum_f(a); b = wave_sum_f(b); c = wave_sum_i(c); d = wave_sum_i(d);
  if (lane == 0) { s.f[w] = a; s.f[4 + w] = b; s.i[w] = c; s.i[4 + w] = d; }
  __syncthreads();
  a = ((s.f[0] + s.f[1]) + s.f[2]) + s.f[3];
  b = ((s.f[4] + s.f[5]) + s.f[6]) + s.f[7];
  c = s.i[0] + s.i[1] + s.i[2] + s.i[3];
  d = s.i[4] + s.i[5] + s.i[6] + s.i[7];
  __syncthreads();
}

__device__ __forceinline__ float block_max_fast(float v, BlockScratch& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_max_f(v);
  if (lane == 0) s.f[8 + w] = v;
  __syncthreads();
  v = fmaxf(fmaxf(s.f[8], s.f[9]), fmaxf(s.f[10], s.f[11]));
  __syncthreads();
  return v;
}

__device__ __forceinline__ float block_sum_fast(float v, BlockScratch& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_sum_f(v);
  if (lane == 0) s.f[12 + w] = v;
  __syncthreads();
  v = ((s.f[12] + s.f[13]) + s.f[14]) + s.f[15];
  __syncthreads();
  return v;
}

__device__ __forceinline__ int block_isum_fast(int v, BlockScratch& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_sum_i(v);
  if (lane == 0) s.i[8 + w] = v;
  __syncthreads();
  v = s.i[8] + s.i[9] + s.i[10] + s.i[11];
  __syncthreads();
  return v;
}

// Exclusive prefix sum of v over the threads in index order; *total gets
// the sum over the block.
__device__ __forceinline__ int block_excl_scan(int v, BlockScratch& s, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) s.wsum[w] = x;
  __syncthreads();
  int before = 0;
  for (int i = 0; i < w; ++i) before += s.wsum[i];
  *total = s.wsum[0] + s.wsum[1] + s.wsum[2] + s.wsum[3];
  __syncthreads();
  return before + x - v;
}

}  // namespace carekv
