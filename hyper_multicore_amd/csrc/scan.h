// Block-wide exclusive scan for 1024-thread blocks over up to 4096 int64 elements in LDS.
#pragma once
#include "common.h"

// Exclusive scan of vals[0..n) in place (LDS array), returns total. blockDim.x must be 1024.
MI355_DEV int64_t block_exclusive_scan_1024(int64_t* vals, int n, int64_t* warp_sums /*[16]*/) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // each thread owns 4 consecutive elements
  int64_t local[4];
  int64_t sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int idx = tid * 4 + i;
    local[i] = idx < n ? vals[idx] : 0;
    sum += local[i];
  }
  // inclusive wave scan of per-thread sums
  int64_t incl = sum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int64_t o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) warp_sums[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int64_t ws = lane < 16 ? warp_sums[lane] : 0;
    int64_t wi = ws;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      int64_t o = __shfl_up(wi, off, 64);
      if (lane >= off) wi += o;
    }
    if (lane < 16) warp_sums[lane] = wi - ws;  // exclusive wave offsets
    if (lane == 15) warp_sums[16] = wi;         // total
  }
  __syncthreads();
  int64_t run = warp_sums[wave] + incl - sum;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int idx = tid * 4 + i;
    if (idx < n) vals[idx] = run;
    run += local[i];
  }
  int64_t total = warp_sums[16];
  __syncthreads();
  return total;
}
