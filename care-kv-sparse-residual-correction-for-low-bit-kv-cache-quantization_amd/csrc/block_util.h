// Work-group (256 threads, 4 waves) reductions and scans with a fixed
// combination order, so results do not depend on scheduling.
#pragma once

#include "common.h"

namespace carekv {

constexpr int kBlock = 256;

struct BlockScratch {
  float f[kBlock];
  int i[kBlock];
  int wsum[4];
  int bc[8];
};

__device__ __forceinline__ float block_sum(float v, BlockScratch& s) {
  s.f[threadIdx.x] = v;
  __syncthreads();
  for (int o = kBlock / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) s.f[threadIdx.x] += s.f[threadIdx.x + o];
    __syncthreads();
  }
  const float r = s.f[0];
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_max(float v, BlockScratch& s) {
  s.f[threadIdx.x] = v;
  __syncthreads();
  for (int o = kBlock / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) s.f[threadIdx.x] = fmaxf(s.f[threadIdx.x], s.f[threadIdx.x + o]);
    __syncthreads();
  }
  const float r = s.f[0];
  __syncthreads();
  return r;
}

__device__ __forceinline__ int block_isum(int v, BlockScratch& s) {
  s.i[threadIdx.x] = v;
  __syncthreads();
  for (int o = kBlock / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) s.i[threadIdx.x] += s.i[threadIdx.x + o];
    __syncthreads();
  }
  const int r = s.i[0];
  __syncthreads();
  return r;
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
