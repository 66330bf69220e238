// Read-bandwidth ceiling of one MI355X for loads issued from the CUs (measurement only; not part of
// the product library). Two families of streaming kernels read a buffer once and discard the data:
//   rc_regs<U>: every lane keeps U 16-byte global loads in flight and folds them into a register
//     (grid-stride over the buffer, any number of waves per CU);
//   rc_lds<U, D>: 8 waves per workgroup, one workgroup per CU (the grouped GEMMs' shape): every wave
//     copies U KB per step straight into LDS (global_load_lds_dwordx4, 1 KB per instruction) into a
//     ring of D steps and waits only for the step issued D - 1 steps earlier.
// The folded value is stored only when it equals a constant the data never produces, so the loads
// cannot be removed and the kernels write nothing in practice.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void rc_regs(const u4* __restrict__ p, int64_t n16, u4* sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  u4 acc = {0, 0, 0, 0};
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    u4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= p[i];
  if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == 0x85ebca6bu && acc.w == 0xc2b2ae35u)
    sink[blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0)
               : "memory", "m0");
}

template <int N> __device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// Step s of wave w of workgroup b covers the U KB at ((s * grid + b) * 8 + w) * U KB.
template <int U, int D>
__global__ __launch_bounds__(512, 1) void rc_lds(const uint8_t* __restrict__ p, int64_t steps, uint4* sink) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  const uint32_t wbase = lds0 + (uint32_t)wave * (uint32_t)(U * D * 1024);
  int64_t s = 0;
  auto issue = [&](int64_t step, int slot) {
    const int64_t chunk = (step * gridDim.x + blockIdx.x) * 8 + wave;
    const uint8_t* base = p + chunk * (int64_t)(U * 1024);
    const uint64_t v = (uint64_t)(uintptr_t)base;
    const uint8_t* ub = (const uint8_t*)(uintptr_t)(((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
                                                    __builtin_amdgcn_readfirstlane((uint32_t)v));
#pragma unroll
    for (int u = 0; u < U; ++u)
      dma16(ub, (uint32_t)(u * 1024 + lane * 16), __builtin_amdgcn_readfirstlane(wbase + (uint32_t)((slot * U + u) * 1024)));
  };
  // prologue: D - 1 steps in flight
  for (; s < D - 1 && s < steps; ++s) issue(s, (int)(s % D));
  for (int64_t q = 0; q < steps; ++q) {
    if (s < steps) { issue(s, (int)(s % D)); ++s; wait_vm<U * (D - 1)>(); }
    else wait_vm<0>();
  }
  wait_vm<0>();
  uint32_t x = *(volatile __attribute__((address_space(3))) uint32_t*)(smem + (threadIdx.x * 16) % (U * D * 1024 * 8));
  if (x == 0x9e3779b9u && lane == 63) sink[blockIdx.x] = make_uint4(x, 0, 0, 0);
}

template <int U, int D>
int launch_lds(const void* p, int64_t bytes, int grid, void* sink, hipStream_t st) {
  const int64_t per_step = (int64_t)grid * 8 * U * 1024;
  const int64_t steps = bytes / per_step;
  const int lds = U * D * 1024 * 8;
  if (steps <= 0 || lds > 160 * 1024) return -1;
  if (hipFuncSetAttribute((const void*)rc_lds<U, D>, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
    return -2;
  hipLaunchKernelGGL((rc_lds<U, D>), dim3(grid), dim3(512), lds, st, (const uint8_t*)p, steps, (uint4*)sink);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

template <int U>
int launch_regs(const void* p, int64_t bytes, int grid, void* sink, hipStream_t st) {
  hipLaunchKernelGGL((rc_regs<U>), dim3(grid), dim3(256), 0, st, (const u4*)p, bytes / 16, (u4*)sink);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // namespace

extern "C" {

// Bytes a run of read_ceiling_lds reads (whole steps of the ring kernel).
int64_t read_ceiling_lds_bytes(int64_t bytes, int grid, int kb_per_step) {
  const int64_t per_step = (int64_t)grid * 8 * kb_per_step * 1024;
  return per_step > 0 ? (bytes / per_step) * per_step : 0;
}

// Register loads: `unroll` 16-byte loads in flight per lane, `grid` workgroups of 256 threads.
// sink: at least grid * 256 * 16 bytes. Returns 0 or a negative error.
int read_ceiling_regs(const void* buf, int64_t bytes, int grid, int unroll, void* sink, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  switch (unroll) {
    case 1: return launch_regs<1>(buf, bytes, grid, sink, st);
    case 2: return launch_regs<2>(buf, bytes, grid, sink, st);
    case 4: return launch_regs<4>(buf, bytes, grid, sink, st);
    case 8: return launch_regs<8>(buf, bytes, grid, sink, st);
    default: return -4;
  }
}

// Direct-to-LDS copies: 8 waves per workgroup, `kb_per_step` KB per wave and step, a ring of `depth`
// steps. sink: at least grid * 16 bytes.
int read_ceiling_lds(const void* buf, int64_t bytes, int grid, int kb_per_step, int depth, void* sink, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  const int key = kb_per_step * 10 + depth;
  switch (key) {
    case 41: return launch_lds<4, 1>(buf, bytes, grid, sink, st);
    case 42: return launch_lds<4, 2>(buf, bytes, grid, sink, st);
    case 44: return launch_lds<4, 4>(buf, bytes, grid, sink, st);
    case 81: return launch_lds<8, 1>(buf, bytes, grid, sink, st);
    case 82: return launch_lds<8, 2>(buf, bytes, grid, sink, st);
    case 21: return launch_lds<2, 1>(buf, bytes, grid, sink, st);
    case 22: return launch_lds<2, 2>(buf, bytes, grid, sink, st);
    case 24: return launch_lds<2, 4>(buf, bytes, grid, sink, st);
    case 28: return launch_lds<2, 8>(buf, bytes, grid, sink, st);
    case 18: return launch_lds<1, 8>(buf, bytes, grid, sink, st);
    default: return -4;
  }
}

}  // extern "C"
