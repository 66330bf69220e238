// Dispatch metadata, token permute and combine (unpermute) for gfx950.
//
// Dispatch is three stream-ordered launches with no host round trip:
//   1. hist:    one wavefront per contiguous chunk of routed slots builds an LDS histogram with
//               LDS atomics and writes its per-chunk counts (no global atomics, so the result is
//               independent of scheduling).
//   2. scan:    one 1024-thread block turns the per-chunk counts into per-expert totals, the
//               exclusive expert offsets, the inclusive group_list and, in place, each chunk's
//               starting rank inside every expert.
//   3. permute: each chunk wavefront replays its slots in order; lanes routed to the same
//               expert in one 64-slot round are ranked with ballots, which keeps the
//               permutation stable (slot order is preserved inside an expert).
// Reference semantics: bincount (modules/mega_moe/route.py:186-211), EP=1 metadata
// (route.py:309-390), permutation convention (tests/ut/examples/moe/test_native_experts.py:59-80,
// ops/common/mega_moe/utilities.asc:176-204), unpermute (route.py:1029-1051).
#pragma clang fp contract(off)
#include "common.h"
#include "scan.h"
#include "decode_prep.h"
#include "gemm.h"
#include "../../include/mi355moe.h"

#define DISPATCH_MAX_EXPERTS 4096
// hist / permute read a chunk's ids in pieces of this many slots, all loads of a piece issued before
// the piece is counted or ranked (a chunk is a multiple of 64 slots; a piece is 16 rounds of 64)
#define DISPATCH_PIECE 1024

struct DispatchPlan {
  int64_t slots;
  int64_t chunk;
  int32_t chunks;
};

static DispatchPlan make_dispatch_plan(int64_t num_tokens, int32_t top_k) {
  DispatchPlan p;
  p.slots = num_tokens * (int64_t)top_k;
  // about 128 chunks (one wavefront each), at least 256 slots (4 rounds of 64) per chunk
  int64_t chunk = (p.slots + 127) / 128;
  chunk = ((chunk + 63) / 64) * 64;
  if (chunk < 256) chunk = 256;
  p.chunk = chunk;
  p.chunks = (int32_t)((p.slots + chunk - 1) / chunk);
  if (p.chunks < 1) p.chunks = 1;
  return p;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" size_t mi355moe_dispatch_workspace_size(int64_t num_tokens, int32_t top_k,
                                                   int32_t num_experts) {
  DispatchPlan p = make_dispatch_plan(num_tokens, top_k);
  // per-chunk counts [chunks][E] + expert starts [E] (int32)
  return align256((size_t)p.chunks * num_experts * 4) + align256((size_t)num_experts * 4);
}

// The ids of slots p0 + 64 r + lane (r < DISPATCH_PIECE / 64) of a chunk ending at `end`: all loads
// issued first (slots past the end re-read the chunk's last slot; callers skip them), then int64 ids
// outside the int32 range become -1 (invalid).
template <typename IdT>
MI355_DEV void load_piece(const IdT* ids, int64_t p0, int64_t end, int lane, int (&idv)[DISPATCH_PIECE / 64]) {
  IdT raw[DISPATCH_PIECE / 64];
#pragma unroll
  for (int r = 0; r < DISPATCH_PIECE / 64; ++r) {
    const int64_t s = p0 + r * 64 + lane;
    raw[r] = ids[s < end ? s : end - 1];
  }
#pragma unroll
  for (int r = 0; r < DISPATCH_PIECE / 64; ++r) {
    const int64_t v = (int64_t)raw[r];
    idv[r] = (v < INT32_MIN || v > INT32_MAX) ? -1 : (int)v;
  }
}

template <typename IdT>
__global__ __launch_bounds__(64) void dispatch_hist_kernel(const IdT* ids, int64_t slots,
                                                           int64_t chunk, int E, int32_t* chunk_counts,
                                                           int32_t* error_flag) {
  extern __shared__ int32_t hist[];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) hist[e] = 0;
  __syncthreads();
  const int64_t begin = (int64_t)blockIdx.x * chunk;
  const int64_t end = begin + chunk < slots ? begin + chunk : slots;
  bool bad = false;
  for (int64_t p0 = begin; p0 < end; p0 += DISPATCH_PIECE) {
    int idv[DISPATCH_PIECE / 64];  // the piece's ids, loaded before they are counted
    load_piece(ids, p0, end, lane, idv);
#pragma unroll
    for (int r = 0; r < DISPATCH_PIECE / 64; ++r) {
      if (p0 + r * 64 + lane >= end) continue;  // past the chunk
      const int id = idv[r];
      if (id >= 0 && id < E) atomicAdd(&hist[id], 1);
      else bad = true;
    }
  }
  if (bad && error_flag != nullptr) error_flag[0] = 1;
  __syncthreads();
  int32_t* out = chunk_counts + (int64_t)blockIdx.x * E;
  for (int e = lane; e < E; e += 64) out[e] = hist[e];
}

// With tile_prefix: also the grouped GEMM's tile plan at tile height bm (tile_prefix[e] = m-tiles of
// the experts before e, [E] = all), which mi355_plan_tiles would compute from group_list.
__global__ __launch_bounds__(1024) void dispatch_scan_kernel(int32_t* chunk_counts, int chunks, int E,
                                                             int32_t* counts, int64_t* expert_offsets,
                                                             int64_t* group_list, int32_t* expert_start,
                                                             int32_t* tile_prefix, int bm) {
  __shared__ int64_t vals[DISPATCH_MAX_EXPERTS];
  __shared__ int32_t tiles[DISPATCH_MAX_EXPERTS];
  __shared__ int64_t wsum[17];
  for (int e = threadIdx.x; e < E; e += 1024) {
    int32_t run = 0;
    for (int b0 = 0; b0 < chunks; b0 += 16) {  // 16 chunk counts loaded at a time, then ranked
      int32_t c[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) c[j] = b0 + j < chunks ? chunk_counts[(int64_t)(b0 + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (b0 + j >= chunks) break;
        chunk_counts[(int64_t)(b0 + j) * E + e] = run;
        run += c[j];
      }
    }
    vals[e] = run;
    if (counts != nullptr) counts[e] = run;
  }
  __syncthreads();
  block_exclusive_scan_1024(vals, E, wsum);
  for (int e = threadIdx.x; e < E; e += 1024) {
    int64_t start = vals[e];
    int64_t cnt = (e + 1 < E ? vals[e + 1] : wsum[16]) - start;
    if (expert_offsets != nullptr) expert_offsets[e] = start;
    if (group_list != nullptr) group_list[e] = start + cnt;
    expert_start[e] = (int32_t)start;
    tiles[e] = cnt > 0 ? (int32_t)((cnt + bm - 1) / bm) : 0;
  }
  if (tile_prefix == nullptr) return;  // block-uniform
  __syncthreads();  // every thread is done with vals
  for (int e = threadIdx.x; e < E; e += 1024) vals[e] = tiles[e];
  __syncthreads();
  const int64_t total = block_exclusive_scan_1024(vals, E, wsum);
  for (int e = threadIdx.x; e < E; e += 1024) tile_prefix[e] = (int32_t)vals[e];
  if (threadIdx.x == 0) tile_prefix[E] = (int32_t)total;
}

template <typename IdT>
__global__ __launch_bounds__(64) void dispatch_permute_kernel(const IdT* ids, int64_t slots,
                                                              int64_t chunk, int E,
                                                              const int32_t* chunk_base,
                                                              const int32_t* expert_start,
                                                              int32_t* mapping, int32_t* gather_index) {
  extern __shared__ int32_t running[];
  const int lane = threadIdx.x;
  const int32_t* base = chunk_base + (int64_t)blockIdx.x * E;
  for (int e = lane; e < E; e += 64) running[e] = expert_start[e] + base[e];
  __syncthreads();
  const int64_t begin = (int64_t)blockIdx.x * chunk;
  const int64_t end = begin + chunk < slots ? begin + chunk : slots;
  int bits = 1;
  while ((1 << bits) < E) ++bits;
  const uint64_t lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
  for (int64_t p0 = begin; p0 < end; p0 += DISPATCH_PIECE) {
  int idv[DISPATCH_PIECE / 64];  // the piece's ids, loaded before its rounds
  load_piece(ids, p0, end, lane, idv);
#pragma unroll
  for (int r = 0; r < DISPATCH_PIECE / 64; ++r) {
    const int64_t s0 = p0 + r * 64;
    if (s0 >= end) break;  // wave-uniform
    const int64_t s = s0 + lane;
    const int id = s < end ? idv[r] : -1;
    bool valid = id >= 0 && id < E;
    uint64_t match = __ballot(valid);
    for (int b = 0; b < bits; ++b) {
      bool bit = valid && ((id >> b) & 1);
      uint64_t m1 = __ballot(bit);
      match &= bit ? m1 : ~m1;
    }
    // The block is one wavefront, whose LDS operations run in program order: every lane reads its
    // expert's running rank before the first lane of each expert advances it. Compiler-only
    // barriers keep that order; a workgroup barrier would also wait for this round's global stores.
    int dest = -1;
    if (valid) dest = running[id] + __popcll(match & lt);
    __builtin_amdgcn_wave_barrier();
    if (valid && (match & lt) == 0) running[id] += __popcll(match);
    __builtin_amdgcn_wave_barrier();
    if (s < end) {
      mapping[s] = dest;
      if (valid && gather_index != nullptr) gather_index[dest] = (int32_t)s;
    }
  }
  }
}

// Internal: enqueue the three dispatch launches. expert_start_ws/chunk_ws come from workspace. With
// tile_prefix, the scan also writes the grouped GEMM's tile plan at tile height bm.
static int dispatch_enqueue(const void* ids, int dtype, int64_t num_tokens, int top_k, int E, int32_t* counts,
                            int64_t* expert_offsets, int64_t* group_list, int32_t* mapping, int32_t* gather_index,
                            int32_t* error_flag, void* workspace, int32_t* tile_prefix, int bm, hipStream_t stream) {
  DispatchPlan p = make_dispatch_plan(num_tokens, top_k);
  int32_t* chunk_counts = (int32_t*)workspace;
  int32_t* expert_start = (int32_t*)((char*)workspace + align256((size_t)p.chunks * E * 4));
  size_t lds = (size_t)E * 4;
  if (dtype == MI355MOE_IDS_INT64)
    hipLaunchKernelGGL(dispatch_hist_kernel<int64_t>, dim3(p.chunks), dim3(64), lds, stream, (const int64_t*)ids,
                       p.slots, p.chunk, E, chunk_counts, error_flag);
  else
    hipLaunchKernelGGL(dispatch_hist_kernel<int32_t>, dim3(p.chunks), dim3(64), lds, stream, (const int32_t*)ids,
                       p.slots, p.chunk, E, chunk_counts, error_flag);
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(1024), 0, stream, chunk_counts, p.chunks, E,
                     counts, expert_offsets, group_list, expert_start, tile_prefix, bm > 0 ? bm : 1);
  if (p.slots > 0 && dtype == MI355MOE_IDS_INT64)
    hipLaunchKernelGGL(dispatch_permute_kernel<int64_t>, dim3(p.chunks), dim3(64), lds, stream, (const int64_t*)ids,
                       p.slots, p.chunk, E, chunk_counts, expert_start, mapping, gather_index);
  else if (p.slots > 0)
    hipLaunchKernelGGL(dispatch_permute_kernel<int32_t>, dim3(p.chunks), dim3(64), lds, stream, (const int32_t*)ids,
                       p.slots, p.chunk, E, chunk_counts, expert_start, mapping, gather_index);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

int mi355_dispatch_enqueue(const void* ids, int dtype, int64_t num_tokens, int top_k, int E, int32_t* counts,
                           int64_t* expert_offsets, int64_t* group_list, int32_t* mapping, int32_t* gather_index,
                           int32_t* error_flag, void* workspace, hipStream_t stream) {
  return dispatch_enqueue(ids, dtype, num_tokens, top_k, E, counts, expert_offsets, group_list, mapping, gather_index,
                          error_flag, workspace, nullptr, 0, stream);
}

int mi355_dispatch_plan_enqueue(const void* ids, int dtype, int64_t num_tokens, int top_k, int E, int32_t* counts,
                                int64_t* group_list, int32_t* mapping, int32_t* gather_index, int32_t* error_flag,
                                void* workspace, int32_t* tile_prefix, int bm, hipStream_t stream) {
  return dispatch_enqueue(ids, dtype, num_tokens, top_k, E, counts, nullptr, group_list, mapping, gather_index,
                          error_flag, workspace, tile_prefix, bm, stream);
}

extern "C" int mi355moe_dispatch(const MI355MoeDispatchArgs* args, void* workspace, size_t workspace_size,
                                 void* stream) {
  if (args == nullptr) return MI355MOE_EINVAL;
  const MI355MoeDispatchArgs& a = *args;
  if (a.num_tokens < 0 || a.top_k <= 0 || a.num_experts <= 0 || a.num_experts > DISPATCH_MAX_EXPERTS)
    return MI355MOE_EINVAL;
  if (a.ids_dtype != MI355MOE_IDS_INT32 && a.ids_dtype != MI355MOE_IDS_INT64) return MI355MOE_EINVAL;
  if ((a.topk_ids == nullptr || a.mapping == nullptr) && a.num_tokens > 0) return MI355MOE_EINVAL;
  if (a.num_tokens * (int64_t)a.top_k > INT32_MAX) return MI355MOE_EINVAL;
  size_t need = mi355moe_dispatch_workspace_size(a.num_tokens, a.top_k, a.num_experts);
  if (workspace == nullptr || workspace_size < need) return -4;
  return mi355_dispatch_enqueue(a.topk_ids, a.ids_dtype, a.num_tokens, a.top_k, a.num_experts, a.counts,
                                a.expert_offsets, a.group_list, a.mapping, a.gather_index, a.error_flag,
                                workspace, (hipStream_t)stream);
}

// The decode prologue in one launch (decode_prep.h): workgroup 0 the dispatch, the others the MX
// token quantisation.
template <bool I64>
__global__ __launch_bounds__(dprep::THREADS) void decode_prep_kernel(dprep::Args a) {
  __shared__ dprep::Lds s;
  dprep::Dev o;
  dprep::run(o, a, I64, s, (int)blockIdx.x);
}

int mi355_decode_prep_enqueue(const dprep::Args& a, int dtype, hipStream_t stream) {
  if (!dprep::applies(a.slots, a.E) || a.mapping == nullptr) return MI355MOE_EINVAL;
  if (a.rows > 0 && (a.cols <= 0 || a.cols % 32 || a.x == nullptr || a.q == nullptr || a.scale == nullptr ||
                     a.scale_ld < a.cols / 32))
    return MI355MOE_EINVAL;
  const int64_t wg = 1 + (a.rows > 0 ? dprep::quant_workgroups(a.rows, a.cols) : 0);
  if (wg > INT32_MAX) return MI355MOE_EINVAL;
  if (dtype == MI355MOE_IDS_INT64)
    hipLaunchKernelGGL(decode_prep_kernel<true>, dim3((unsigned)wg), dim3(dprep::THREADS), 0, stream, a);
  else
    hipLaunchKernelGGL(decode_prep_kernel<false>, dim3((unsigned)wg), dim3(dprep::THREADS), 0, stream, a);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// routed[mapping[s]] = x[s / K], 16-byte vectors; one block row per slot.
__global__ __launch_bounds__(256) void permute_rows_kernel(const uint16_t* x, int64_t slots, int K, int H,
                                                           const int32_t* mapping, uint16_t* routed) {
  const int64_t s = blockIdx.x;
  if (s >= slots) return;
  const int32_t dest = mapping[s];
  if (dest < 0) return;
  const int64_t t = s / K;
  const uint4* src = (const uint4*)(x + t * (int64_t)H);
  uint4* dst = (uint4*)(routed + (int64_t)dest * H);
  for (int v = threadIdx.x; v < H / 8; v += blockDim.x) dst[v] = src[v];
}

// Zero `bytes` (a multiple of 16, 16-byte aligned) with a fill kernel: stream-ordered like a memset
// and safe to record in a captured graph.
__global__ __launch_bounds__(256) void zero16_kernel(uint4* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

int mi355_zero_enqueue(void* p, size_t bytes, hipStream_t st) {
  if (bytes == 0) return MI355MOE_OK;
  if (p == nullptr || bytes % 16 || ((uintptr_t)p & 15)) return MI355MOE_EINVAL;
  const int64_t n = (int64_t)(bytes / 16);
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(zero16_kernel, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, st, (uint4*)p, n);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

int mi355_permute_rows_enqueue(const uint16_t* x, int64_t slots, int K, int H, const int32_t* mapping,
                                uint16_t* routed, hipStream_t st) {
  if (slots == 0) return MI355MOE_OK;
  hipLaunchKernelGGL(permute_rows_kernel, dim3((unsigned)slots), dim3(H >= 2048 ? 256 : 64), 0, st, x, slots, K, H,
                     mapping, routed);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

extern "C" int mi355moe_token_permute(const uint16_t* x, int64_t num_tokens, int32_t hidden_size,
                                      const void* topk_ids, int32_t ids_dtype, int32_t top_k,
                                      int32_t num_experts, uint16_t* routed, int32_t* mapping,
                                      void* workspace, size_t workspace_size, void* stream) {
  if (num_tokens < 0 || hidden_size <= 0 || hidden_size % 8 || top_k <= 0 || num_experts <= 0 ||
      num_experts > DISPATCH_MAX_EXPERTS)
    return MI355MOE_EINVAL;
  if (ids_dtype != MI355MOE_IDS_INT32 && ids_dtype != MI355MOE_IDS_INT64) return MI355MOE_EINVAL;
  if (num_tokens > 0 && (x == nullptr || topk_ids == nullptr || routed == nullptr || mapping == nullptr))
    return MI355MOE_EINVAL;
  if (num_tokens * (int64_t)top_k > INT32_MAX) return MI355MOE_EINVAL;
  size_t need = mi355moe_dispatch_workspace_size(num_tokens, top_k, num_experts);
  if (workspace == nullptr || workspace_size < need) return -4;
  hipStream_t st = (hipStream_t)stream;
  int rc = mi355_dispatch_enqueue(topk_ids, ids_dtype, num_tokens, top_k, num_experts, nullptr, nullptr,
                                  nullptr, mapping, nullptr, nullptr, workspace, st);
  if (rc) return rc;
  int64_t slots = num_tokens * top_k;
  if (slots > 0)
    hipLaunchKernelGGL(permute_rows_kernel, dim3((unsigned)slots), dim3(hidden_size >= 2048 ? 256 : 64), 0, st,
                       x, slots, top_k, hidden_size, mapping, routed);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

// out[t] = bf16(sum_k p[t,k] * y[mapping[t*K+k]]) with fp32 accumulation in ascending k; the
// product and the sum are rounded separately (no fma), so the result is reproducible bit for bit.
// Block (t, c): token t, columns 8 * 128 c .. of it, each thread one 16-byte vector (8 columns), so a
// decode batch of few tokens still spreads over many workgroups. The K rows' vectors are loaded four
// at a time before they are added (in ascending k).
constexpr int UNPERMUTE_THREADS = 128;
__global__ __launch_bounds__(UNPERMUTE_THREADS) void unpermute_kernel(const uint16_t* y, const int32_t* mapping,
                                                                      const float* probs, int64_t T, int K, int H,
                                                                      uint16_t* out) {
  const int64_t t = blockIdx.x;
  if (t >= T) return;
  __shared__ int32_t rows[64];
  __shared__ float ps[64];
  if (threadIdx.x < K) {
    rows[threadIdx.x] = mapping[t * K + threadIdx.x];
    ps[threadIdx.x] = probs != nullptr ? probs[t * K + threadIdx.x] : 1.0f;
  }
  __syncthreads();
  const int v = blockIdx.y * UNPERMUTE_THREADS + threadIdx.x;
  if (v >= H / 8) return;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 4) {
    uint4 q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int32_t r = k0 + j < K ? rows[k0 + j] : -1;
      q[j] = r >= 0 ? ((const uint4*)(y + (int64_t)r * H))[v] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (k0 + j >= K || rows[k0 + j] < 0) continue;
      const float p = ps[k0 + j];
      const uint32_t w[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = acc[2 * i] + p * bf16_to_f32((uint16_t)(w[i] & 0xffff));
        acc[2 * i + 1] = acc[2 * i + 1] + p * bf16_to_f32((uint16_t)(w[i] >> 16));
      }
    }
  }
  uint4 o;
  o.x = f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
  o.y = f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
  o.z = f32_to_bf16(acc[4]) | ((uint32_t)f32_to_bf16(acc[5]) << 16);
  o.w = f32_to_bf16(acc[6]) | ((uint32_t)f32_to_bf16(acc[7]) << 16);
  ((uint4*)(out + t * (int64_t)H))[v] = o;
}

int mi355_unpermute_enqueue(const uint16_t* y, const int32_t* mapping, const float* probs, int64_t T, int K,
                            int H, uint16_t* out, hipStream_t stream) {
  if (T == 0) return MI355MOE_OK;
  if (T > INT32_MAX) return MI355MOE_EINVAL;
  const dim3 grid((unsigned)T, (unsigned)((H / 8 + UNPERMUTE_THREADS - 1) / UNPERMUTE_THREADS));
  hipLaunchKernelGGL(unpermute_kernel, grid, dim3(UNPERMUTE_THREADS), 0, stream, y, mapping, probs, T, K, H, out);
  return hipGetLastError() == hipSuccess ? MI355MOE_OK : MI355MOE_ELAUNCH;
}

extern "C" int mi355moe_token_unpermute(const uint16_t* y, const int32_t* mapping, const float* probs,
                                        int64_t num_tokens, int32_t top_k, int32_t hidden_size,
                                        uint16_t* out, void* stream) {
  if (num_tokens < 0 || top_k <= 0 || top_k > 64 || hidden_size <= 0 || hidden_size % 8) return MI355MOE_EINVAL;
  if (num_tokens > 0 && (y == nullptr || mapping == nullptr || out == nullptr)) return MI355MOE_EINVAL;
  return mi355_unpermute_enqueue(y, mapping, probs, num_tokens, top_k, hidden_size, out, (hipStream_t)stream);
}
