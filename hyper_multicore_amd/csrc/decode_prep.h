// Decode prologue of the MegaMoE forward in one launch: the dispatch (expert histogram, scan, group
// list, tile plan and stable permutation) in workgroup 0, and the MX token quantisation in the other
// workgroups.
//
// At decode shapes (T * K routed slots of a few thousand) the three dispatch kernels of dispatch.hip
// and the token quantisation are four launches that each do a few microseconds of work; here they
// are one. Workgroup 0 (256 threads, 4 wavefronts) does what dispatch.hip's hist / scan / permute do
// with one wavefront per quarter of the slots instead of one per chunk:
//   1. hist:    wave w counts its quarter's slots into its own LDS histogram row with LDS atomics;
//   2. scan:    thread e turns the 4 rows of column e into the rows' starting ranks inside expert e
//               (the per-wave bases) and the expert total; a block scan gives the exclusive expert
//               starts, the inclusive group_list and, at tile height bm, the tile plan;
//   3. permute: wave w replays its quarter in slot order and ranks the lanes routed to one expert in
//               a 64-slot round with ballots (slot order is kept inside an expert).
// The result is the unique stable counting sort, so it equals the three-launch dispatch exactly.
// Workgroups 1.. quantise the token rows [T, H] (one thread per 32-column block, row-major scales),
// as mx_quant_rows_kernel does; the decode GEMMs read tokens through the gather index, so the
// quantisation does not wait for the dispatch.
//
// The code is written against a policy O (thread index, barriers, ballots, shuffles, LDS atomics,
// the e4m3 conversion): the kernel in dispatch.hip uses the device one; the tests run the same code
// under a host emulation of a workgroup (one thread per lane, barriers for the lockstep points).
// Reference semantics: bincount (modules/mega_moe/route.py:186-211), EP=1 metadata
// (route.py:309-390), permutation convention (ops/common/mega_moe/utilities.asc:176-204), token
// quantisation (ops/common/mega_moe/adapters/arch35/quantization/dual_axis_mxfp8_worker.h:39-66).
#pragma once
#include "common.h"

namespace dprep {

constexpr int THREADS = 256;
constexpr int WAVES = THREADS / 64;
constexpr int MAX_EXPERTS = 1024;
constexpr int64_t MAX_SLOTS = 8192;  // at most 2048 slots (32 rounds of 64) per wavefront
constexpr int PER_THREAD = MAX_EXPERTS / THREADS;  // scan elements per thread

struct Args {
  const void* ids;       // [slots] int32 or int64 expert ids
  int64_t slots;         // T * K
  int E;
  int32_t* counts;       // [E] or null
  int64_t* group_list;   // [E] inclusive ends, or null
  int32_t* mapping;      // [slots] slot -> routed row (-1 for an invalid id)
  int32_t* gather;       // [slots] routed row -> slot, or null
  int32_t* error_flag;   // set to 1 for an id outside [0, E), or null
  int32_t* tile_prefix;  // [E + 1] m-tiles before each expert at tile height bm, or null
  int bm;
  // token quantisation (workgroups 1..): x [rows, cols] bf16 -> q [rows, cols] e4m3, scale
  // [rows, scale_ld] e8m0; rows = 0 for none
  const uint16_t* x;
  int64_t rows;
  int cols;
  uint8_t* q;
  uint8_t* scale;
  int64_t scale_ld;
};

struct Lds {
  int32_t hist[WAVES][MAX_EXPERTS];  // per-wave counts, then per-wave running ranks
  int32_t tiles[MAX_EXPERTS];
  int64_t vals[MAX_EXPERTS];
  int64_t wsum[WAVES + 1];
};

// Workgroups of the launch: 1 for the dispatch and one per 256 token blocks.
inline int64_t quant_workgroups(int64_t rows, int cols) { return (rows * (cols / 32) + THREADS - 1) / THREADS; }

// Whether the one-launch prologue takes a dispatch of this size.
inline bool applies(int64_t slots, int E) { return slots > 0 && slots <= MAX_SLOTS && E >= 1 && E <= MAX_EXPERTS; }

// Quarter of the slots owned by wave w: [begin, end), a multiple of 64 slots long except the last.
MI355_HD void quarter(int64_t slots, int w, int64_t& begin, int64_t& end) {
  int64_t q = (slots + WAVES - 1) / WAVES;
  q = (q + 63) / 64 * 64;
  begin = w * q < slots ? w * q : slots;
  end = begin + q < slots ? begin + q : slots;
}

MI355_HD int load_id(const Args& a, bool i64, int64_t s) {
  const int64_t v = i64 ? ((const int64_t*)a.ids)[s] : (int64_t)((const int32_t*)a.ids)[s];
  return (v < 0 || v >= a.E) ? -1 : (int)v;  // -1 also for int64 ids outside the int32 range
}

// Exclusive scan of vals[0..n) (n <= MAX_EXPERTS) in place over the workgroup; returns the total.
// Thread t owns elements PER_THREAD * t ..; wave-inclusive scan by shuffles, then the 4 wave sums.
template <class O>
MI355_HD int64_t block_scan(O& o, int64_t* vals, int n, int64_t* wsum) {
  const int tid = o.tid(), lane = tid & 63, wave = tid >> 6;
  int64_t local[PER_THREAD];
  int64_t sum = 0;
  for (int i = 0; i < PER_THREAD; ++i) {
    const int idx = tid * PER_THREAD + i;
    local[i] = idx < n ? vals[idx] : 0;
    sum += local[i];
  }
  int64_t incl = sum;
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t v = o.shfl_up(incl, off);
    if (lane >= off) incl += v;
  }
  if (lane == 63) wsum[wave] = incl;
  o.sync();
  if (tid == 0) {
    int64_t run = 0;
    for (int w = 0; w < WAVES; ++w) {
      const int64_t v = wsum[w];
      wsum[w] = run;
      run += v;
    }
    wsum[WAVES] = run;
  }
  o.sync();
  int64_t run = wsum[wave] + incl - sum;
  for (int i = 0; i < PER_THREAD; ++i) {
    const int idx = tid * PER_THREAD + i;
    if (idx < n) vals[idx] = run;
    run += local[i];
  }
  const int64_t total = wsum[WAVES];
  o.sync();  // every thread has read wsum before a later scan writes it
  return total;
}

// Workgroup 0: the dispatch. All 256 threads reach every barrier; ballots and shuffles are in
// wave-uniform control flow.
template <class O>
MI355_HD void dispatch(O& o, const Args& a, bool i64, Lds& s) {
  const int tid = o.tid(), lane = tid & 63, w = tid >> 6;
  const int E = a.E;
  for (int e = tid; e < E; e += THREADS)
    for (int v = 0; v < WAVES; ++v) s.hist[v][e] = 0;
  o.sync();
  int64_t begin, end;
  quarter(a.slots, w, begin, end);
  // 1. histogram of the wave's quarter
  bool bad = false;
  for (int64_t s0 = begin; s0 < end; s0 += 64) {
    const int64_t sl = s0 + lane;
    if (sl >= end) continue;
    const int id = load_id(a, i64, sl);
    if (id >= 0) o.lds_add(&s.hist[w][id], 1);
    else bad = true;
  }
  if (bad && a.error_flag != nullptr) a.error_flag[0] = 1;
  o.sync();
  // 2. per-expert totals and per-wave bases, then the expert starts
  for (int e = tid; e < E; e += THREADS) {
    int32_t run = 0;
    for (int v = 0; v < WAVES; ++v) {
      const int32_t c = s.hist[v][e];
      s.hist[v][e] = run;
      run += c;
    }
    s.vals[e] = run;
    if (a.counts != nullptr) a.counts[e] = run;
  }
  o.sync();
  const int64_t total = block_scan(o, s.vals, E, s.wsum);
  const int bm = a.bm > 0 ? a.bm : 1;
  for (int e = tid; e < E; e += THREADS) {
    const int64_t start = s.vals[e];
    const int64_t cnt = (e + 1 < E ? s.vals[e + 1] : total) - start;
    if (a.group_list != nullptr) a.group_list[e] = start + cnt;
    s.tiles[e] = cnt > 0 ? (int32_t)((cnt + bm - 1) / bm) : 0;
    for (int v = 0; v < WAVES; ++v) s.hist[v][e] += (int32_t)start;  // running ranks of each wave
  }
  o.sync();
  if (a.tile_prefix != nullptr) {  // workgroup-uniform
    for (int e = tid; e < E; e += THREADS) s.vals[e] = s.tiles[e];
    o.sync();
    const int64_t tiles = block_scan(o, s.vals, E, s.wsum);
    for (int e = tid; e < E; e += THREADS) a.tile_prefix[e] = (int32_t)s.vals[e];
    if (tid == 0) a.tile_prefix[E] = (int32_t)tiles;
  }
  // 3. stable permutation of the wave's quarter (the wave's running ranks are its own LDS row)
  int bits = 1;
  while ((1 << bits) < E) ++bits;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int32_t* running = s.hist[w];
  for (int64_t s0 = begin; s0 < end; s0 += 64) {  // wave-uniform
    const int64_t sl = s0 + lane;
    const int id = sl < end ? load_id(a, i64, sl) : -1;
    const bool valid = id >= 0;
    uint64_t match = o.ballot(valid);
    for (int b = 0; b < bits; ++b) {
      const bool bit = valid && ((id >> b) & 1);
      const uint64_t m1 = o.ballot(bit);
      match &= bit ? m1 : ~m1;
    }
    // every lane reads its expert's running rank before the expert's first lane advances it
    int dest = -1;
    if (valid) dest = running[id] + o.popc(match & lt);
    o.wave_sync();
    if (valid && (match & lt) == 0) running[id] += o.popc(match);
    o.wave_sync();
    if (sl < end) {
      a.mapping[sl] = dest;
      if (valid && a.gather != nullptr) a.gather[dest] = (int32_t)sl;
    }
  }
}

// One 32-column block b of token row r: e4m3 elements and the block's e8m0 code, as
// mx_quant_rows_kernel writes them (row-major scales).
template <class O>
MI355_HD void quant_block(O& o, const Args& a, int64_t r, int b) {
  const uint8_t* src = (const uint8_t*)(a.x + r * a.cols + b * 32);
  float v[32];
  for (int i = 0; i < 4; ++i) {
    uint32_t u[4];
    o.load16(src + 16 * i, u);
    for (int j = 0; j < 4; ++j) {
      v[i * 8 + 2 * j] = bf16_to_f32((uint16_t)(u[j] & 0xffff));
      v[i * 8 + 2 * j + 1] = bf16_to_f32((uint16_t)(u[j] >> 16));
    }
  }
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const uint32_t code = mx_scale_code(amax);
  uint32_t out[8];
  for (int i = 0; i < 8; ++i)
    out[i] = o.e4m3(mx_apply_inv_scale(v[4 * i], code)) | (o.e4m3(mx_apply_inv_scale(v[4 * i + 1], code)) << 8) |
             (o.e4m3(mx_apply_inv_scale(v[4 * i + 2], code)) << 16) |
             (o.e4m3(mx_apply_inv_scale(v[4 * i + 3], code)) << 24);
  o.store16(a.q + r * a.cols + b * 32, out[0], out[1], out[2], out[3]);
  o.store16(a.q + r * a.cols + b * 32 + 16, out[4], out[5], out[6], out[7]);
  a.scale[r * a.scale_ld + b] = (uint8_t)code;
}

// The whole launch: workgroup `wg` of 1 + quant_workgroups(rows, cols).
template <class O>
MI355_HD void run(O& o, const Args& a, bool i64, Lds& s, int wg) {
  if (wg == 0) {
    dispatch(o, a, i64, s);
    return;
  }
  const int nb = a.cols / 32;
  const int64_t id = (int64_t)(wg - 1) * THREADS + o.tid();
  if (id >= a.rows * nb) return;
  const int64_t r = id / nb;
  quant_block(o, a, r, (int)(id - r * nb));
}

// Device policy.
struct Dev {
  MI355_DEV int tid() const { return (int)threadIdx.x; }
  MI355_DEV void sync() const { __syncthreads(); }
  // the wavefront's LDS operations run in program order: a compiler-only barrier keeps that order
  MI355_DEV void wave_sync() const { __builtin_amdgcn_wave_barrier(); }
  MI355_DEV uint64_t ballot(bool p) const { return __ballot(p); }
  MI355_DEV int64_t shfl_up(int64_t v, int off) const { return __shfl_up(v, off, 64); }
  MI355_DEV int popc(uint64_t m) const { return __popcll(m); }
  MI355_DEV void lds_add(int32_t* p, int32_t v) const { atomicAdd(p, v); }
  MI355_DEV uint32_t e4m3(float v) const { return f32_to_e4m3_inrange(v); }
  MI355_DEV void load16(const uint8_t* p, uint32_t (&u)[4]) const {
    const uint4 v = *(const uint4*)p;
    u[0] = v.x, u[1] = v.y, u[2] = v.z, u[3] = v.w;
  }
  MI355_DEV void store16(uint8_t* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) const {
    *(uint4*)p = make_uint4(a, b, c, d);
  }
};

}  // namespace dprep
