// Host-side copy checker for the grouped GEMM (test infrastructure; never runs on a GPU).
//
// The library's host code (api.hip, backward.hip, dispatch.hip, quant.hip, gemm.hip compiled for the
// host only, with every optional path switched on) is linked against this file, which supplies:
//   * stand-ins for the HIP runtime entry points the host code calls (kernel launches do nothing,
//     hipMemsetAsync writes host memory), so all "device" buffers are plain host allocations;
//   * host versions of the internal enqueue functions whose results later stages read (dispatch
//     metadata, tile prefix) and of the grouped GEMM launches, which, instead of launching, run the
//     GEMM's copy schedule on the host for every work item, wave and lane: the same copy-plan code
//     and issue functions the kernels compile (gemm_plan.h and its .inc fragments), with a recorder
//     as the copy instruction.
// Every recorded copy is checked for:
//   1. its global source lying inside one live allocation (16 or 4 bytes per lane);
//   2. its LDS destination lying inside the ring slot of its stage (below the tile prefix);
//   3. its source being exactly the element the LDS fragment reads expect at that LDS position,
//      computed from the tensor shapes of the C-ABI call (independently of the GGParams the host
//      code built) for rows and columns that reach the output;
//   4. the vmcnt wait before each stage leaving only loads younger than that stage in flight, and
//      every ring slot being refilled only after the stage it held has been read;
//   5. full coverage of each stage's weight slot (and scale slots) by the four waves.
// The epilogue's output ranges are checked against the output allocation, and every host-side read
// of the index arrays runs under AddressSanitizer; UndefinedBehaviorSanitizer ends the run at any report.
//
// Usage: gemm_copy_check [scenario-name ...]   (no argument: all scenarios). Exit status 0 when
// every check passed.
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "../../hyper_multicore_amd/csrc/gemm_plan.h"
#include "../../include/mi355moe.h"

// ------------------------------------------------------------------------------------------------
// Allocations and error reporting
struct Alloc {
  uint8_t* p;
  size_t n;
  std::string name;
};
static std::vector<Alloc> g_allocs;
static long g_errors = 0, g_copies = 0, g_items = 0, g_gemms = 0;
static std::string g_scenario;
// Use the 256-row tiles even where the library would pick the 64-row ones (the state of a build with
// the decode tiles switched off): planning and launch both follow it.
static bool g_force_big = false;
// The forward tile-configuration variant the scenario passes through the C ABI (gemm_variant
// argument / MI355MoeForwardArgs::gemm_variant).
static int g_variant = 0;

#define CHECK_FAIL(...)                                         \
  do {                                                          \
    if (g_errors < 30) {                                        \
      fprintf(stderr, "[%s] ", g_scenario.c_str());             \
      fprintf(stderr, __VA_ARGS__);                             \
      fputc('\n', stderr);                                      \
    }                                                           \
    ++g_errors;                                                 \
  } while (0)

static uint8_t* mk(const char* name, size_t n, int fill = 0x5a) {
  uint8_t* p = (uint8_t*)malloc(n ? n : 1);
  if (!p) {
    fprintf(stderr, "out of memory (%s, %zu bytes)\n", name, n);
    exit(2);
  }
  memset(p, fill, n);
  g_allocs.push_back({p, n, name});
  return p;
}
static void free_all() {
  for (auto& a : g_allocs) free(a.p);
  g_allocs.clear();
}
// The host stand-in of the library's static device array (`scratch` of the no-allocation entry point):
// hipGetSymbolAddress answers this address, which stays valid for the whole run, as the device array
// does for the process.
alignas(256) static uint8_t g_symbol_scratch[(MI355MOE_NOALLOC_MAX_GROUPS + 1) * 4];
static const Alloc g_symbol_alloc = {g_symbol_scratch, sizeof(g_symbol_scratch), "scratch (static device array)"};
static const Alloc* find_alloc(const void* q, size_t sz) {
  const uint8_t* b = (const uint8_t*)q;
  for (const auto& a : g_allocs)
    if (b >= a.p && b + sz <= a.p + a.n) return &a;
  if (b >= g_symbol_alloc.p && b + sz <= g_symbol_alloc.p + g_symbol_alloc.n) return &g_symbol_alloc;
  return nullptr;
}
static const Alloc* alloc_of(const void* q) { return find_alloc(q, 1); }

// ------------------------------------------------------------------------------------------------
// HIP runtime stand-ins (the host code only enqueues; nothing here touches a GPU)
static long g_launches = 0;
extern "C" {
void** __hipRegisterFatBinary(const void*) {
  static void* handle = nullptr;
  return &handle;
}
void __hipRegisterFunction(void**, const void*, char*, const char*, unsigned int, uint3*, uint3*, dim3*, dim3*, int*) {}
void __hipUnregisterFatBinary(void**) {}
void __hipRegisterVar(void**, void*, char*, const char*, int, size_t, int, int) {}
static long g_symbol_lookups = 0;
hipError_t hipGetSymbolAddress(void** ptr, const void*) {
  ++g_symbol_lookups;
  *ptr = g_symbol_scratch;
  return hipSuccess;
}
hipError_t __hipPushCallConfiguration(dim3, dim3, size_t, hipStream_t) { return hipSuccess; }
hipError_t __hipPopCallConfiguration(dim3* g, dim3* b, size_t* s, hipStream_t* st) {
  *g = dim3(1);
  *b = dim3(1);
  *s = 0;
  *st = nullptr;
  return hipSuccess;
}
hipError_t hipLaunchKernel(const void*, dim3, dim3, void**, size_t, hipStream_t) {
  ++g_launches;
  return hipSuccess;
}
hipError_t hipMemsetAsync(void* dst, int value, size_t n, hipStream_t) {
  if (n && !find_alloc(dst, n)) {
    CHECK_FAIL("hipMemsetAsync of %zu bytes outside every allocation", n);
    return hipErrorInvalidValue;
  }
  memset(dst, value, n);
  return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
hipError_t hipGetLastError(void) { return hipSuccess; }
hipError_t hipFuncSetAttribute(const void*, hipFuncAttribute, int) { return hipSuccess; }
hipError_t hipGetDevice(int* d) {
  *d = 0;
  return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
  *v = 256;
  return hipSuccess;
}
}

// ------------------------------------------------------------------------------------------------
// Host versions of the enqueue functions whose outputs the GEMM set-up reads
int mi355_plan_tiles(const int64_t* group_list, int G, int32_t* tile_prefix, hipStream_t, bool small) {
  if (g_force_big) small = false;
  const int bm = mi355_gg_bm(small);
  if (!find_alloc(tile_prefix, (size_t)(G + 1) * 4)) CHECK_FAIL("tile prefix of %d groups outside its buffer", G);
  int64_t acc = 0;
  for (int g = 0; g < G; ++g) {
    const int64_t rows = group_list[g] - (g ? group_list[g - 1] : 0);
    tile_prefix[g] = (int32_t)acc;
    acc += rows > 0 ? (rows + bm - 1) / bm : 0;
  }
  tile_prefix[G] = (int32_t)acc;
  return MI355MOE_OK;
}

int mi355_plan_row_blocks(const int64_t* group_list, int G, int rows, int32_t* prefix, hipStream_t) {
  if (!find_alloc(prefix, (size_t)(G + 1) * 4)) CHECK_FAIL("block prefix of %d groups outside its buffer", G);
  int64_t acc = 0;
  for (int g = 0; g < G; ++g) {
    const int64_t n = group_list[g] - (g ? group_list[g - 1] : 0);
    prefix[g] = (int32_t)acc;
    acc += n > 0 ? (n + rows - 1) / rows : 0;
  }
  prefix[G] = (int32_t)acc;
  return MI355MOE_OK;
}

// The routed-row MX quantisation (quant.hip mx_quant_grouped_kernel) replayed for its addresses: every
// block's reads of its source and writes of data and scales must stay inside their allocations, and
// the launch must cover every planned block.
static void check_span(const void* base, int64_t lo, int64_t hi, const char* what) {
  if (hi > lo && !find_alloc((const uint8_t*)base + lo, (size_t)(hi - lo)))
    CHECK_FAIL("%s: bytes %lld..%lld outside every allocation", what, (long long)lo, (long long)hi);
}
int mi355_mx_quant_grouped(const MxGroupedQuant& q, hipStream_t) {
  if (q.R <= 0) return MI355MOE_OK;
  if (q.C <= 0 || q.C % 32 || q.G <= 0 || q.group_list == nullptr || q.block_prefix == nullptr) return MI355MOE_EINVAL;
  const int64_t max_blocks = (q.R + 31) / 32 + q.G;
  if (q.block_prefix[q.G] > max_blocks) CHECK_FAIL("planned %d row blocks, launch covers %lld", q.block_prefix[q.G],
                                                   (long long)max_blocks);
  for (int g = 0; g < q.G; ++g) {
    const int64_t start = g ? q.group_list[g - 1] : 0, n = q.group_list[g] - start;
    for (int64_t b = 0; 32 * b < n; ++b) {
      const int64_t r0 = start + 32 * b, nrows = std::min<int64_t>(32, n - 32 * b);
      for (int64_t i = 0; i < nrows; ++i) {
        const int64_t r = r0 + i;
        if (q.mode == MX_Q_BF16) {
          const int64_t sr = q.gather ? q.gather[r] / q.gather_div : r;
          check_span(q.src, sr * q.src_ld * 2, (sr * q.src_ld + q.C) * 2, "quant source row");
        } else if (q.mode == MX_Q_SWIGLU) {
          check_span(q.U, r * 2 * q.C * 2, (r + 1) * 2 * q.C * 2, "quant U row");
        } else {
          check_span(q.U, r * q.C * 2, (r + 1) * q.C * 2, "quant U row");
          check_span(q.da, r * (q.C / 2) * 2, (r + 1) * (q.C / 2) * 2, "quant gA row");
        }
        if (q.row_data) {
          check_span(q.row_data, r * q.C, (r + 1) * q.C, "row-axis data");
          check_span(q.row_scale, r * q.row_scale_ld, r * q.row_scale_ld + q.C / 32, "row-axis scales");
        }
        if (q.col_data) check_span(q.col_data, r * q.C, (r + 1) * q.C, "column-axis data");
      }
      if (q.col_data) {
        const int64_t pair = (start / 64 + g + b / 2) * q.C * 2;
        check_span(q.col_scale, pair, pair + (int64_t)q.C * 2, "column-axis scales");
      }
    }
  }
  return MI355MOE_OK;
}

// Stable counting sort of the T*K slots by expert id (the dispatch contract of include/mi355moe.h).
int mi355_dispatch_enqueue(const void* ids, int dtype, int64_t T, int K, int E, int32_t* counts, int64_t* offsets,
                           int64_t* group_list, int32_t* mapping, int32_t* gather, int32_t* error_flag, void*,
                           hipStream_t) {
  const int64_t S = T * K;
  std::vector<int64_t> c(E, 0);
  auto id_of = [&](int64_t s) -> int64_t {
    return dtype == MI355MOE_IDS_INT64 ? ((const int64_t*)ids)[s] : (int64_t)((const int32_t*)ids)[s];
  };
  bool bad = false;
  for (int64_t s = 0; s < S; ++s) {
    const int64_t e = id_of(s);
    if (e < 0 || e >= E) bad = true;
    else ++c[e];
  }
  std::vector<int64_t> start(E, 0);
  for (int e = 1; e < E; ++e) start[e] = start[e - 1] + c[e - 1];
  for (int e = 0; e < E; ++e) {
    if (counts) counts[e] = (int32_t)c[e];
    if (offsets) offsets[e] = start[e];
    if (group_list) group_list[e] = start[e] + c[e];
  }
  std::vector<int64_t> next = start;
  for (int64_t s = 0; s < S; ++s) {
    const int64_t e = id_of(s);
    const int64_t r = (e < 0 || e >= E) ? -1 : next[e]++;
    if (mapping) mapping[s] = (int32_t)r;
    if (gather && r >= 0) gather[r] = (int32_t)s;
  }
  if (error_flag && bad) *error_flag = 1;
  return MI355MOE_OK;
}

// The dispatch with the tile plan: the two host versions above and below, in that order.
int mi355_dispatch_plan_enqueue(const void* ids, int dtype, int64_t T, int K, int E, int32_t* counts,
                                int64_t* group_list, int32_t* mapping, int32_t* gather, int32_t* error_flag,
                                void* ws, int32_t* tile_prefix, int bm, hipStream_t st) {
  const int rc = mi355_dispatch_enqueue(ids, dtype, T, K, E, counts, nullptr, group_list, mapping, gather,
                                        error_flag, ws, st);
  if (rc) return rc;
  return mi355_plan_tiles(group_list, E, tile_prefix, st, bm == mi355_gg_bm(true));
}
// The one-launch decode prologue: the kernel's own code (decode_prep.h) under the host emulation of
// prep_sim.inc, checked against the host dispatch above and the host tile plan. Under g_force_big the
// plan is then rewritten at the 256-row height the GEMM replays assume.
#include "prep_sim.inc"
static long g_preps = 0;
int mi355_decode_prep_enqueue(const dprep::Args& a, int dtype, hipStream_t st) {
  if (!dprep::applies(a.slots, a.E) || a.mapping == nullptr) return MI355MOE_EINVAL;
  const bool i64 = dtype == MI355MOE_IDS_INT64;
  check_span(a.ids, 0, a.slots * (i64 ? 8 : 4), "decode prologue ids");
  check_span(a.mapping, 0, a.slots * 4, "decode prologue mapping");
  if (a.gather) check_span(a.gather, 0, a.slots * 4, "decode prologue gather");
  if (a.counts) check_span(a.counts, 0, (int64_t)a.E * 4, "decode prologue counts");
  if (a.group_list) check_span(a.group_list, 0, (int64_t)a.E * 8, "decode prologue group_list");
  if (a.tile_prefix) check_span(a.tile_prefix, 0, (int64_t)(a.E + 1) * 4, "decode prologue tile plan");
  if (a.rows > 0) {
    check_span(a.x, 0, a.rows * a.cols * 2, "decode prologue tokens");
    check_span(a.q, 0, a.rows * a.cols, "decode prologue e4m3 tokens");
    check_span(a.scale, 0, (a.rows - 1) * a.scale_ld + a.cols / 32, "decode prologue token scales");
  }
  if (prep_sim::run(a, i64) != 0) return MI355MOE_EINVAL;
  ++g_preps;
  // the host dispatch and plan on copies
  const int E = a.E;
  std::vector<int32_t> counts(E), mapping(a.slots), gather(a.slots, -1), prefix(E + 1);
  std::vector<int64_t> gl(E);
  const int T = (int)a.slots;  // the host dispatch takes T * K slots: K = 1
  mi355_dispatch_enqueue(a.ids, dtype, T, 1, E, counts.data(), nullptr, gl.data(), mapping.data(), gather.data(),
                         nullptr, nullptr, st);
  for (int e = 0, run = 0; e < E; ++e) {
    prefix[e] = run;
    run += (int)((counts[e] + a.bm - 1) / a.bm);
    prefix[E] = run;
  }
  if (memcmp(mapping.data(), a.mapping, a.slots * 4)) CHECK_FAIL("decode prologue: mapping differs");
  const int64_t routed = gl[E - 1];
  if (a.gather && memcmp(gather.data(), a.gather, routed * 4)) CHECK_FAIL("decode prologue: gather differs");
  if (a.counts && memcmp(counts.data(), a.counts, E * 4)) CHECK_FAIL("decode prologue: counts differ");
  if (a.group_list && memcmp(gl.data(), a.group_list, E * 8)) CHECK_FAIL("decode prologue: group_list differs");
  if (a.tile_prefix && memcmp(prefix.data(), a.tile_prefix, (E + 1) * 4)) CHECK_FAIL("decode prologue: tile plan differs");
  if (a.tile_prefix && g_force_big && a.group_list) return mi355_plan_tiles(a.group_list, E, a.tile_prefix, st, false);
  return MI355MOE_OK;
}
int mi355_zero_enqueue(void* p, size_t bytes, hipStream_t) {
  if (bytes && !find_alloc(p, bytes)) {
    CHECK_FAIL("zero fill of %zu bytes outside every allocation", bytes);
    return MI355MOE_EINVAL;
  }
  if (bytes % 16 || ((uintptr_t)p & 15)) return MI355MOE_EINVAL;
  memset(p, 0, bytes);
  return MI355MOE_OK;
}
int mi355_permute_rows_enqueue(const uint16_t*, int64_t, int, int, const int32_t*, uint16_t*, hipStream_t) {
  return MI355MOE_OK;
}
int mi355_unpermute_enqueue(const uint16_t*, const int32_t*, const float*, int64_t, int, int, uint16_t*, hipStream_t) {
  return MI355MOE_OK;
}
int mi355_mx_quant_rows(const uint16_t*, int64_t, int, uint8_t*, uint8_t*, int64_t, hipStream_t) {
  return MI355MOE_OK;
}

// ------------------------------------------------------------------------------------------------
// Expected operand layout: where the element the LDS reads expect lives, from the shapes of the
// C-ABI call. A scenario that knows the operands of a GEMM sets `g_expect` before the call; GEMMs on
// the library's internal buffers fall back to the addressing implied by their GGParams, and are
// then still bounds-checked against the allocations.
struct Expect {
  bool set = false;
  const uint8_t* A = nullptr;  // [rowsA, Kd] elements, row stride a_row_bytes
  int64_t a_row_bytes = 0;
  const uint8_t* a_scale = nullptr;  // MX: [rowsA, a_scale_ld] codes
  int64_t a_scale_ld = 0;
  const uint8_t* B = nullptr;  // [G, Kd, Ntot] (EIO) or [G, Ntot, Kd] (EOI) elements
  const uint8_t* b_scale = nullptr;  // MX EIO: [G, Kd/64, Ntot, 2]; MX EOI: [G, Ntot, b_scale_ld]
  int64_t b_scale_ld = 0;
};
static Expect g_expect;

struct Layout {
  const uint8_t* A;
  int64_t a_row_bytes;
  const int32_t* gather;
  int gather_div;
  const uint8_t* as;
  int64_t as_ld;
  const uint8_t* B;
  bool eoi;
  int64_t Kd, Ntot;
  int esize;
  const uint8_t* bs;
  int64_t bs_ld;
  int64_t src_row(int64_t routed) const { return gather ? gather[routed] / gather_div : routed; }
  const uint8_t* a_at(int64_t routed, int64_t kbyte) const { return A + src_row(routed) * a_row_bytes + kbyte; }
  const uint8_t* b_at(int g, int64_t k, int64_t col) const {
    const int64_t e = eoi ? ((int64_t)g * Ntot + col) * Kd + k : ((int64_t)g * Kd + k) * Ntot + col;
    return B + e * esize;
  }
  const uint8_t* as_at(int64_t routed, int64_t code) const { return as + src_row(routed) * as_ld + code; }
  // MX EIO col_scale [G, Kd/64, Ntot, 2]: the two codes of column col for the 64-K group kg
  const uint8_t* bs_col_at(int g, int64_t kg, int64_t col) const { return bs + (((int64_t)g * (Kd / 64) + kg) * Ntot + col) * 2; }
  // MX EOI row scales [G, Ntot, bs_ld]
  const uint8_t* bs_row_at(int g, int64_t col, int64_t code) const { return bs + ((int64_t)g * Ntot + col) * bs_ld + code; }
};

// Tile column n (0 .. BN-1) of n-tile nt -> weight column; false when its output column is past N.
// (SwiGLU: each WN-wide wave tile holds WN/2 gate columns and then the WN/2 matching up columns.
// With `gu` the weight stores gate and up columns in alternating 64-column blocks: output column o
// has its gate column in block 2 (o / 64) and its up column in block 2 (o / 64) + 1.)
template <class C>
static bool tile_weight_col(int n, int nt, int N, bool swiglu, int gu, int64_t* wcol) {
  if (!swiglu) {
    const int64_t o = (int64_t)nt * C::BN + n;
    *wcol = o;
    return o < N;
  }
  const int H = C::WN / 2, q = n / C::WN, jj = n % C::WN;
  const int64_t o = (int64_t)nt * (C::BN / 2) + q * H + (jj % H);
  if (gu)
    *wcol = (o / 64) * 128 + (jj < H ? 0 : 64) + o % 64;
  else
    *wcol = jj < H ? o : N + o;
  return o < N;
}

// ------------------------------------------------------------------------------------------------
// The recorder used as the copy instruction
struct Rec {
  const uint8_t* g;
  int sz;
  uint32_t off;
  int iter;  // pipelined step whose barrier preceded the copy (-1: before the K loop)
};
struct Wait {
  size_t pos;  // copies recorded before the wait
  int stage;   // stage read after the following barrier
  int n;       // loads allowed in flight
};
static std::vector<Rec>* g_rec = nullptr;
static int g_iter = -1;
struct CheckDma {
  template <int SZ>
  static void copy(const void* g, uint32_t off, uint8_t*, int enable) {
    if (!enable) return;
    g_rec->push_back({(const uint8_t*)g, SZ, off, g_iter});
  }
};

// R_ASS: grouped-K MX only - the per-stage column scales of A, A_SLOTS slots of 512 bytes at AS_OFF
enum Region { R_A = 0, R_B, R_BS, R_AS, R_BSR, R_ASS, R_N };
static const char* region_name(int r) {
  static const char* n[] = {"A", "B", "B-scale", "A-scale", "B-row-scale", "A-column-scale"};
  return n[r];
}

// One lane's copy sequence of one work item, replayed in the K loop's order (k_loop in gemm.hip:
// prologue, the wait for stage 0, then for every pipelined step k the wait for stage k + 1 and the
// copy items of the step).
template <class C, bool MX, bool B_KN, bool LA, bool GK>
static void record_schedule(const CopyPlan<C>& cp, int nk, int wave, std::vector<Rec>& rec, std::vector<Wait>& waits) {
  uint8_t* smem = nullptr;
  g_rec = &rec;
  g_iter = -1;
  {
    using D = CheckDma;
#include "../../hyper_multicore_amd/csrc/gemm_kloop_prologue.inc"
    waits.push_back({rec.size(), 0, younger_than<C, LA>(0, -1, nk, la_n, lb_n)});
    for (int k = 0; k < nk - 1; ++k) {
      waits.push_back({rec.size(), k + 1, younger_than<C, LA>(k + 1, k - 1, nk, la_n, lb_n)});
      g_iter = k;
      for (int it = 0; it < StepShape<C, MX, 1, GK>::ITEMS; ++it)
        issue_item<C, MX, B_KN, LA, GK, D>(cp, k, nk, wave, smem, it);
      issue_scales_item<C, MX, B_KN, LA, D, GK>(cp, k, nk, wave, smem);
    }
  }
  g_rec = nullptr;
}

// Per work item bookkeeping shared by the lanes
struct ItemCtx {
  int g, nt, split, nk;
  int half = -1;      // forward: the column half of the tile the item computes (-1: all of it)
  int64_t tile_row0;  // forward: first routed row; grouped-K: unused
  int rows_valid;
  // grouped-K
  int k0, kend, m0;
  std::vector<uint8_t> cov[R_N];  // coverage bitmaps [stage or group][slot bytes]
};

struct Decoded {
  int region, slot, stage;  // stage (A/B/BS) or scale group (AS/BSR)
  uint32_t rel;             // byte offset of this lane's data inside the slot
};

template <class C>
static bool classify(uint32_t pos, int sz, Decoded& d, bool gk_mx) {
  if (pos + sz > (uint32_t)C::PREFIX_OFF) return false;
  if (gk_mx && pos >= (uint32_t)C::AS_OFF && pos < (uint32_t)C::BSR_OFF) {
    const uint32_t q = pos - C::AS_OFF;
    d.region = R_ASS;
    d.slot = q / C::BS_BYTES;
    d.rel = q % C::BS_BYTES;
    return d.rel + sz <= (uint32_t)C::BS_BYTES;
  }
  if (pos < (uint32_t)C::B_OFF) {
    d.region = R_A;
    d.slot = pos / C::A_BYTES;
    d.rel = pos % C::A_BYTES;
    return d.rel + sz <= (uint32_t)C::A_BYTES;
  }
  if (pos < (uint32_t)C::AS_OFF) {
    const uint32_t q = pos - C::B_OFF;
    d.slot = q / C::B_SLOT;
    const uint32_t rel = q % C::B_SLOT;
    if (rel < (uint32_t)C::B_BYTES) {
      d.region = R_B;
      d.rel = rel;
      return rel + sz <= (uint32_t)C::B_BYTES;
    }
    d.region = R_BS;
    d.rel = rel - C::B_BYTES;
    return d.rel + sz <= (uint32_t)C::BS_BYTES;
  }
  if (pos < (uint32_t)C::BSR_OFF) {
    const uint32_t q = pos - C::AS_OFF;
    d.region = R_AS;
    d.slot = q / C::AS_SLOT;
    d.rel = q % C::AS_SLOT;
    return d.rel + sz <= (uint32_t)C::AS_SLOT;
  }
  const uint32_t q = pos - C::BSR_OFF;
  d.region = R_BSR;
  d.slot = q / C::BSR_SLOT;
  d.rel = q % C::BSR_SLOT;
  return d.slot < 2 && d.rel + sz <= (uint32_t)C::BSR_SLOT;
}

// The element the fragment reads expect at LDS byte `rel` of a slot of `region` holding `stage`,
// or nullptr when that position feeds only rows / columns the epilogue drops.
template <class C, bool MX, bool B_KN, bool SWIGLU, bool GK>
static const uint8_t* expected_src(const GGParams& p, const Layout& L, const ItemCtx& it, int region, int stage,
                                   uint32_t rel, bool* zero_ok) {
  *zero_ok = false;
  int64_t wcol;
  if constexpr (GK) {
    // both operands K-major. bf16: K row k (32 per stage) at k*512, chunk c stored at c ^ ((k&7)<<1),
    // 8 columns per chunk; MX: K row k (64 per stage) at k*256, chunk c at c ^ (k & 15), 16 columns
    constexpr int ES = MX ? 1 : 2;
    constexpr int RB = MX ? 256 : 512;
    if (region == R_BS || region == R_ASS) {  // MX: two codes for each of columns 2m, 2m+1 per stage
      const int64_t grp = (int64_t)(it.k0 / 64) + it.g + stage;
      const int64_t col = (region == R_ASS ? (int64_t)it.m0 : (int64_t)it.nt * C::BN) + (rel / 4) * 2;
      const int64_t cols = region == R_ASS ? p.m_rows : p.N;
      if (col >= cols) return nullptr;
      return (region == R_ASS ? p.a_scale : p.b_scale) + (grp * cols + col) * 2;
    }
    const int k = rel / RB, cpos = (rel % RB) / 16;
    const int c = MX ? (cpos ^ (k & 15)) : (cpos ^ ((k & 7) << 1));
    const int64_t row = (int64_t)it.k0 + (int64_t)stage * (MX ? 64 : 32) + k;
    const int64_t col = (region == R_A ? (int64_t)it.m0 : (int64_t)it.nt * C::BN) + c * (16 / ES);
    if (col >= (region == R_A ? p.m_rows : p.N)) return nullptr;
    if (row >= it.kend) {
      *zero_ok = true;
      return nullptr;
    }
    if (region == R_A) return L.A + row * L.a_row_bytes + col * ES;
    return L.B + row * L.Ntot * ES + col * ES;
  } else {
    const int64_t kstage = (int64_t)it.split * it.nk + stage;  // stage index along the full K
    // a column half: positions of the other half's columns feed only the idle waves
    auto other_half = [&](int n) { return it.half >= 0 && n / (C::BN / 2) != it.half; };
    switch (region) {
      case R_A: {
        const int r = rel / 64, cpos = (rel % 64) / 16, c = cpos ^ ((r >> 2) & 3);
        if (r >= it.rows_valid) return nullptr;
        return L.a_at(it.tile_row0 + r, kstage * C::KB + c * 16);
      }
      case R_B: {
        if (!B_KN) {  // K-contiguous weight rows, laid out like the activations
          const int n = rel / 64, cpos = (rel % 64) / 16, c = cpos ^ ((n >> 2) & 3);
          if (other_half(n)) return nullptr;
          if (!tile_weight_col<C>(n, it.nt, p.N, SWIGLU, p.gate_up_interleaved, &wcol)) return nullptr;
          return L.b_at(it.g, (kstage * C::KB + c * 16) / L.esize, wcol);
        }
        if (MX) {  // 64 K rows of 256 bytes, chunk c at c ^ (k & 15), 16 columns per chunk
          const int k = rel / 256, cpos = (rel % 256) / 16, c = cpos ^ (k & 15);
          if (other_half(c * 16)) return nullptr;
          if (!tile_weight_col<C>(c * 16, it.nt, p.N, SWIGLU, p.gate_up_interleaved, &wcol)) return nullptr;
          return L.b_at(it.g, kstage * 64 + k, wcol);
        }
        // bf16: 32 K rows of 512 bytes, chunk c at c ^ ((k & 7) << 1), 8 columns per chunk
        const int k = rel / 512, cpos = (rel % 512) / 16, c = cpos ^ ((k & 7) << 1);
        if (other_half(c * 8)) return nullptr;
        if (!tile_weight_col<C>(c * 8, it.nt, p.N, SWIGLU, p.gate_up_interleaved, &wcol)) return nullptr;
        return L.b_at(it.g, kstage * 32 + k, wcol);
      }
      case R_BS: {  // two codes for each of tile columns 2m, 2m+1 (4 bytes per lane)
        const int n = (rel / 4) * 2;
        if (other_half(n)) return nullptr;
        if (!tile_weight_col<C>(n, it.nt, p.N, SWIGLU, p.gate_up_interleaved, &wcol)) return nullptr;
        return L.bs_col_at(it.g, kstage, wcol);
      }
      case R_AS: {  // 16 codes (8 stages) per row
        const int r = rel / 16;
        if (r >= it.rows_valid) return nullptr;
        return L.as_at(it.tile_row0 + r, (int64_t)stage * 16);
      }
      case R_BSR: {  // 16 codes (8 stages) per tile column
        const int n = rel / 16;
        if (other_half(n)) return nullptr;
        if (!tile_weight_col<C>(n, it.nt, p.N, SWIGLU, p.gate_up_interleaved, &wcol)) return nullptr;
        return L.bs_row_at(it.g, wcol, (int64_t)stage * 16);
      }
    }
  }
  return nullptr;
}

// Checks one lane's copies of one work item; accumulates the coverage of the item's slots.
template <class C, bool MX, bool B_KN, bool SWIGLU, bool GK>
static void check_lane(const GGParams& p, const Layout& L, ItemCtx& it, int wave, int lane, bool la,
                       const std::vector<Rec>& rec, const std::vector<Wait>& waits) {
  const int slots[R_N] = {C::A_SLOTS, C::B_SLOTS, C::B_SLOTS, 2, 2, C::A_SLOTS};
  const int per_fill[R_N] = {C::A_PER, C::B_PER, 1, 1, 1, 1};
  int fills[R_N][8] = {};
  std::vector<Decoded> dec(rec.size());
  for (size_t i = 0; i < rec.size(); ++i) {
    const Rec& r = rec[i];
    ++g_copies;
    if (!find_alloc(r.g, r.sz)) {
      const Alloc* a = alloc_of(r.g);
      CHECK_FAIL("copy %zu (wave %d lane %d, group %d n-tile %d) reads %d bytes outside every allocation%s%s", i, wave,
                 lane, it.g, it.nt, r.sz, a ? ": past the end of " : "", a ? a->name.c_str() : "");
      continue;
    }
    Decoded& d = dec[i];
    Decoded first_lane, last_lane;
    const uint32_t pos = r.off + (uint32_t)r.sz * lane;
    const bool ok = classify<C>(pos, r.sz, d, GK && MX) && classify<C>(r.off, r.sz, first_lane, GK && MX) &&
                    classify<C>(r.off + 63u * r.sz, r.sz, last_lane, GK && MX) && first_lane.region == last_lane.region &&
                    first_lane.slot == last_lane.slot;
    if (!ok) {
      CHECK_FAIL("copy %zu (wave %d lane %d) writes LDS %u..%u outside one ring slot", i, wave, lane, r.off,
                 r.off + 64u * r.sz);
      d.region = -1;
      continue;
    }
    if (d.slot >= slots[d.region]) {
      CHECK_FAIL("copy %zu writes slot %d of the %s ring (%d slots)", i, d.slot, region_name(d.region), slots[d.region]);
      d.region = -1;
      continue;
    }
    // stage (or scale group) held: slots are filled in stage order, per_fill copies per stage
    const int f = fills[d.region][d.slot]++;
    d.stage = d.slot + slots[d.region] * (f / per_fill[d.region]);
    const bool group = d.region == R_AS || d.region == R_BSR;
    if ((group ? 8 * d.stage : d.stage) >= it.nk) {
      CHECK_FAIL("copy %zu loads %s %s %d of an item with %d stages", i, region_name(d.region), group ? "group" : "stage",
                 d.stage, it.nk);
      continue;
    }
    // ring reuse: the previous occupant of the slot was read in the step before its stage
    const int prev = d.stage - slots[d.region];
    if (prev >= 0) {
      const int prev_last = group ? 8 * prev + 7 : prev;
      if (prev_last > r.iter)
        CHECK_FAIL("copy %zu refills the %s slot of %s %d at step %d while stage %d may still be read", i,
                   region_name(d.region), group ? "group" : "stage", prev, r.iter, prev_last);
    }
    // source element
    bool zero_ok = false;
    const uint8_t* want = expected_src<C, MX, B_KN, SWIGLU, GK>(p, L, it, d.region, d.stage, d.rel, &zero_ok);
    if (zero_ok) {
      const Alloc* z = alloc_of(p.zero_row);
      if (!z || r.g < p.zero_row || r.g + r.sz > p.zero_row + z->n) {
        CHECK_FAIL("grouped-K copy %zu past the group end does not read the zero row", i);
      } else {
        for (int b = 0; b < r.sz; ++b)
          if (r.g[b] != 0) {
            CHECK_FAIL("zero row holds a nonzero byte");
            break;
          }
      }
    } else if (want != nullptr && want != r.g) {
      CHECK_FAIL("copy %zu (wave %d lane %d, group %d n-tile %d, %s %s %d, LDS byte %u) reads %+lld bytes from the "
                 "expected element",
                 i, wave, lane, it.g, it.nt, region_name(d.region), group ? "group" : "stage", d.stage, d.rel,
                 (long long)(r.g - want));
    }
    // coverage
    auto& cov = it.cov[d.region];
    const int unit = d.region == R_A ? C::A_BYTES
                   : d.region == R_B ? C::B_BYTES
                   : d.region == R_BS ? C::BS_BYTES
                   : d.region == R_AS ? C::AS_SLOT : d.region == R_BSR ? C::BSR_SLOT : C::BS_BYTES;
    const size_t base = (size_t)d.stage * unit + d.rel;
    if (base + r.sz <= cov.size())
      for (int b = 0; b < r.sz; ++b) {
        if (cov[base + b]) {
          CHECK_FAIL("LDS byte %u of %s %d written twice", d.rel + b, region_name(d.region), d.stage);
          break;
        }
        cov[base + b] = 1;
      }
  }
  // waits: before the barrier that precedes reading stage j, every load of stage j (and of its
  // scale group) issued by this wave is older than the n loads allowed in flight
  for (const Wait& w : waits) {
    const size_t done = w.pos >= (size_t)w.n ? w.pos - w.n : 0;
    for (size_t i = 0; i < rec.size(); ++i) {
      const Decoded& d = dec[i];
      if (d.region < 0) continue;
      const bool group = d.region == R_AS || d.region == R_BSR;
      const bool needed = group ? d.stage == w.stage / C::AS_GROUP : d.stage == w.stage;
      if (needed && i >= done)
        CHECK_FAIL("wave %d: the wait before stage %d (vmcnt %d after %zu loads) leaves load %zu (%s %d) in flight",
                   wave, w.stage, w.n, w.pos, i, region_name(d.region), d.stage);
    }
  }
  (void)la;
}

// Coverage of one item: every byte of each weight / scale slot a stage reads was written once;
// activation rows inside the tile were written.
template <class C, bool MX, bool B_KN, bool GK>
static void check_coverage(const ItemCtx& it) {
  auto full = [&](int region, int stages, int unit, int used, const char* what) {
    for (int s = 0; s < stages; ++s)
      for (int b = 0; b < used; ++b)
        if (!it.cov[region][(size_t)s * unit + b]) {
          CHECK_FAIL("group %d n-tile %d: byte %d of %s %d never loaded", it.g, it.nt, b, what, s);
          return;
        }
  };
  const int ngroups = (it.nk + C::AS_GROUP - 1) / C::AS_GROUP;
  full(R_B, it.nk, C::B_BYTES, C::B_BYTES, "weight stage");
  if (GK) full(R_A, it.nk, C::A_BYTES, C::A_BYTES, "activation stage");
  else full(R_A, it.nk, C::A_BYTES, it.rows_valid * 64, "activation stage");
  if (MX && B_KN) full(R_BS, it.nk, C::BS_BYTES, C::BS_BYTES, "weight scale stage");
  if (MX && !B_KN) full(R_BSR, ngroups, C::BSR_SLOT, C::BSR_SLOT, "weight row-scale group");
  if (MX && !GK) full(R_AS, ngroups, C::AS_SLOT, it.rows_valid * 16, "activation scale group");
  if (MX && GK) full(R_ASS, it.nk, C::BS_BYTES, C::BS_BYTES, "A column-scale stage");
}

static void check_range(const void* base, int64_t lo, int64_t hi, const char* what) {
  if (hi <= lo) return;
  const uint8_t* b = (const uint8_t*)base;
  if (!find_alloc(b + lo, (size_t)(hi - lo))) CHECK_FAIL("%s writes bytes %lld..%lld outside its allocation", what,
                                                         (long long)lo, (long long)hi);
}

// ------------------------------------------------------------------------------------------------
// Functional emulation of a work item: the copies land in an emulated LDS, the fragment reads and
// MFMAs run through the kernels' own read_elem / mfma_elem with an emulation of the lane-crossing
// instructions (transposing LDS loads, 32x32 MFMAs), and the accumulators are compared with a
// reference GEMM of the same operands. The instruction models: ds_read_b64_tr_b16 - each 16-lane
// group's four 16-bit values per lane form a 4 x 16 block (lane i holds row i / 4, columns
// 4 (i % 4) ..), and lane o receives column o; ds_read_b64_tr_b8 - 8 x 16 bytes (lane i holds row
// i / 2, columns 8 (i % 2) ..); v_mfma_f32_32x32x16_bf16 - lane l holds row / column l % 32 and
// K = 8 (l / 32) + j; v_mfma_scale_f32_32x32x64_f8f6f4 - byte j / 16 + j of lane l holds
// K = 16 (l / 32) + j / 32 + 16 (l / 32) + j, lane r + 32 b supplies the scale of K block b of row /
// column r; accumulator element r of lane l is row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
// Paths that already pass on the GPU (EIO bf16 and MX, EOI bf16) calibrate these models.
static bool g_emulate = false;
static long g_emulated_items = 0;

static float bf16f(uint16_t v) {
  uint32_t u = (uint32_t)v << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static float e4m3f(uint8_t v) {
  const int sign = v >> 7, e = (v >> 3) & 15, m = v & 7;
  float r;
  if (e == 15 && m == 7) r = NAN;
  else if (e == 0) r = std::ldexp((float)m, -9);
  else r = std::ldexp(1.0f + m / 8.0f, e - 7);
  return sign ? -r : r;
}
static float e8m0f(int code) { return std::ldexp(1.0f, (code & 255) - 127); }

struct EmuState {
  int pass = 0;  // 0: record the transposing loads' addresses, 1: replay their results
  int lane = 0, idx = 0;
  std::vector<const uint8_t*> addr;  // [call * 64 + lane]
  std::vector<int> kind;             // per call: 16 (b16) or 8 (b8)
  std::vector<uint64_t> val;         // [call * 64 + lane]
  // MFMA operands of the current call, per lane
  uint8_t a[64][32], b[64][32];
  int sa[64], sb[64];
  v16f* acc[64];
};
static EmuState g_emu;

struct EmuOps {
  static uint64_t take(const uint8_t* p, int kind) {
    EmuState& e = g_emu;
    const size_t slot = (size_t)e.idx * 64 + e.lane;
    if (e.pass == 0) {
      if (e.addr.size() < slot + 1) e.addr.resize((size_t)(e.idx + 1) * 64, nullptr);
      if ((int)e.kind.size() < e.idx + 1) e.kind.resize(e.idx + 1, 0);
      e.addr[slot] = p;
      e.kind[e.idx] = kind;
      ++e.idx;
      return 0;
    }
    ++e.idx;
    return e.val[slot];
  }
  static v4s tr16(const uint8_t* p) {
    const uint64_t v = take(p, 16);
    v4s r;
    memcpy(&r, &v, 8);
    return r;
  }
  static v2i tr8(const uint8_t* p) {
    const uint64_t v = take(p, 8);
    v2i r;
    memcpy(&r, &v, 8);
    return r;
  }
  static void mfma_bf16(v8bf a, v8bf b, v16f& acc) {
    memcpy(g_emu.a[g_emu.lane], &a, 16);
    memcpy(g_emu.b[g_emu.lane], &b, 16);
    g_emu.acc[g_emu.lane] = &acc;
  }
  static void mfma_f8(v8i a, v8i b, v16f& acc, int sa, int sb) {
    memcpy(g_emu.a[g_emu.lane], &a, 32);
    memcpy(g_emu.b[g_emu.lane], &b, 32);
    g_emu.sa[g_emu.lane] = sa;
    g_emu.sb[g_emu.lane] = sb;
    g_emu.acc[g_emu.lane] = &acc;
  }
};

// results of the recorded transposing loads
static void emu_resolve_loads() {
  EmuState& e = g_emu;
  const int calls = (int)e.kind.size();
  e.val.assign((size_t)calls * 64, 0);
  for (int c = 0; c < calls; ++c)
    for (int grp = 0; grp < 4; ++grp) {
      uint8_t in[16][8];
      for (int i = 0; i < 16; ++i) memcpy(in[i], e.addr[(size_t)c * 64 + grp * 16 + i], 8);
      for (int o = 0; o < 16; ++o) {
        uint8_t out[8];
        if (e.kind[c] == 16) {  // 4 x 16 block of 16-bit values
          for (int r = 0; r < 4; ++r) {
            const int lane = 4 * r + o / 4, j = o % 4;
            memcpy(out + 2 * r, in[lane] + 2 * j, 2);
          }
        } else {  // 8 x 16 block of bytes
          for (int r = 0; r < 8; ++r) {
            const int lane = 2 * r + o / 8, j = o % 8;
            out[r] = in[lane][j];
          }
        }
        memcpy(&e.val[(size_t)c * 64 + grp * 16 + o], out, 8);
      }
    }
}

static void emu_resolve_mfma(bool f8) {
  EmuState& e = g_emu;
  float d[32][32];
  for (int row = 0; row < 32; ++row)
    for (int col = 0; col < 32; ++col) {
      double sum = 0.0;
      if (!f8) {
        for (int k = 0; k < 16; ++k) {
          uint16_t av, bv;
          memcpy(&av, e.a[row + 32 * (k / 8)] + 2 * (k % 8), 2);
          memcpy(&bv, e.b[col + 32 * (k / 8)] + 2 * (k % 8), 2);
          sum += (double)bf16f(av) * bf16f(bv);
        }
      } else {
        for (int k = 0; k < 64; ++k) {
          const int half = (k % 32) / 16, byte = (k / 32) * 16 + k % 16, blk = k / 32;
          const float av = e4m3f(e.a[row + 32 * half][byte]) * e8m0f(e.sa[row + 32 * blk]);
          const float bv = e4m3f(e.b[col + 32 * half][byte]) * e8m0f(e.sb[col + 32 * blk]);
          sum += (double)av * bv;
        }
      }
      d[row][col] = (float)sum;
    }
  for (int l = 0; l < 64; ++l)
    for (int r = 0; r < 16; ++r) {
      const int row = 8 * (r / 4) + 4 * (l / 32) + r % 4, col = l % 32;
      (*e.acc[l])[r] += d[row][col];
    }
}

// Copies land in the emulated LDS at once: every read of a slot happens after its stage's copies and
// before the slot is refilled (the copy checks above establish both).
static int g_fill_lane = 0;
struct FillDma {
  template <int SZ>
  static void copy(const void* g, uint32_t off, uint8_t* smem, int enable) {
    if (!enable) return;
    memcpy(smem + off + (uint32_t)SZ * g_fill_lane, g, SZ);
  }
};

template <class C, bool MX, bool B_KN, bool LA, bool GK>
static void fill_prologue(const CopyPlan<C>& cp, int nk, int wave, uint8_t* smem) {
  using D = FillDma;
#include "../../hyper_multicore_amd/csrc/gemm_kloop_prologue.inc"
  (void)la_n;
  (void)lb_n;
}
template <class C, bool MX, bool B_KN, bool LA, bool GK>
static void fill_step(const CopyPlan<C>& cp, int k, int nk, int wave, uint8_t* smem) {
  for (int it = 0; it < StepShape<C, MX, 1, GK>::ITEMS; ++it)
    issue_item<C, MX, B_KN, LA, GK, FillDma>(cp, k, nk, wave, smem, it);
  issue_scales_item<C, MX, B_KN, LA, FillDma, GK>(cp, k, nk, wave, smem);
}

template <class C, bool MX, bool B_KN, bool GK>
struct EmuWaveTile {
  using F = Frags<C, MX, B_KN, GK>;
  F f0[64], f1[64];
  v16f acc[64][C::MI][C::NI];
};

// LDS slot pointers of stage kn, as the K loop computes them
template <class C, bool MX, bool GK>
static void stage_ptrs(uint8_t* smem, int kn, const uint8_t*& As, const uint8_t*& Bs, const uint8_t*& ASs,
                       const uint8_t*& BSRs) {
  As = smem + (kn % C::A_SLOTS) * C::A_BYTES;
  Bs = smem + C::B_OFF + (kn % C::B_SLOTS) * C::B_SLOT;
  if (MX && GK) ASs = smem + C::AS_OFF + (kn % C::A_SLOTS) * C::BS_BYTES;
  else ASs = smem + C::AS_OFF + ((kn / C::AS_GROUP) & 1) * C::AS_SLOT + (kn & (C::AS_GROUP - 1)) * 2;
  BSRs = smem + C::BSR_OFF + ((kn / C::AS_GROUP) & 1) * C::BSR_SLOT + (kn & (C::AS_GROUP - 1)) * 2;
}

template <class C, bool MX, bool B_KN, int NM, bool GK>
static void emu_read_stage(typename EmuWaveTile<C, MX, B_KN, GK>::F (&f)[64], uint8_t* smem, int kn, int wm, int wn) {
  const uint8_t *As, *Bs, *ASs, *BSRs;
  stage_ptrs<C, MX, GK>(smem, kn, As, Bs, ASs, BSRs);
  using SS = StepShape<C, MX, NM, GK>;
  for (int e = 0; e < SS::READS; ++e) {
    g_emu.pass = 0;
    g_emu.addr.clear();
    g_emu.kind.clear();
    typename EmuWaveTile<C, MX, B_KN, GK>::F scratch;
    for (int l = 0; l < 64; ++l) {
      g_emu.lane = l;
      g_emu.idx = 0;
      read_elem<C, MX, B_KN, NM, GK, EmuOps>(scratch, e, As, Bs, ASs, BSRs, wm, wn, l);
    }
    if (!g_emu.kind.empty()) emu_resolve_loads();
    g_emu.pass = 1;
    for (int l = 0; l < 64; ++l) {
      g_emu.lane = l;
      g_emu.idx = 0;
      read_elem<C, MX, B_KN, NM, GK, EmuOps>(f[l], e, As, Bs, ASs, BSRs, wm, wn, l);
    }
  }
}

template <class C, bool MX, bool B_KN, int NM, bool GK>
static void emu_mfma_stage(const typename EmuWaveTile<C, MX, B_KN, GK>::F (&f)[64],
                           v16f (&acc)[64][C::MI][C::NI]) {
  using SS = StepShape<C, MX, NM, GK>;
  for (int t = 0; t < SS::MFMAS; ++t) {
    for (int l = 0; l < 64; ++l) {
      g_emu.lane = l;
      mfma_elem<C, MX, B_KN, NM, GK, EmuOps>(f[l], acc[l], t);
    }
    emu_resolve_mfma(MX);
  }
}

// The K loop of one wave: reads of stage k + 1 and MFMAs of stage k per step, copies of all waves
// applied in iteration order (they never touch a slot that is being read).
template <class C, bool MX, bool B_KN, int NM, bool GK>
static void emu_wave_loop(EmuWaveTile<C, MX, B_KN, GK>& w, uint8_t* smem, int nk, int wm, int wn, int k) {
  if constexpr (NM > 0) {
    if (k < 0) {  // prologue read of stage 0
      emu_read_stage<C, MX, B_KN, NM, GK>(w.f0, smem, 0, wm, wn);
      return;
    }
    auto& cur = (k & 1) ? w.f1 : w.f0;
    auto& nxt = (k & 1) ? w.f0 : w.f1;
    emu_mfma_stage<C, MX, B_KN, NM, GK>(cur, w.acc);
    if (k + 1 < nk) emu_read_stage<C, MX, B_KN, NM, GK>(nxt, smem, k + 1, wm, wn);
  }
}
template <class C, bool MX, bool B_KN, bool GK>
static void emu_wave_step(EmuWaveTile<C, MX, B_KN, GK>& w, int nm, uint8_t* smem, int nk, int wm, int wn, int k) {
  if (C::MI >= 4 && nm == 4) emu_wave_loop<C, MX, B_KN, (C::MI >= 4 ? 4 : 1), GK>(w, smem, nk, wm, wn, k);
  else if (nm == 2) emu_wave_loop<C, MX, B_KN, 2, GK>(w, smem, nk, wm, wn, k);
  else if (nm == 1) emu_wave_loop<C, MX, B_KN, 1, GK>(w, smem, nk, wm, wn, k);
}

// Runs one work item; cps[wave][lane] are the lanes' copy plans. value(row, col) returns the
// reference of accumulator tile element (row, col) or NAN where the tile position is not compared.
template <class C, bool MX, bool B_KN, bool GK>
static void emulate_item(const CopyPlan<C> (&cps)[C::WAVES][64], const bool (&la)[C::WAVES], const int (&nm)[C::WAVES],
                         int nk, const std::function<double(int, int)>& value, const char* what,
                         const std::function<void(const EmuWaveTile<C, MX, B_KN, GK>*)>& epilogue = nullptr) {
  std::vector<uint8_t> lds(C::TOTAL, 0);
  uint8_t* smem = lds.data();
  auto tiles = std::make_unique<EmuWaveTile<C, MX, B_KN, GK>[]>(C::WAVES);
  for (int w = 0; w < C::WAVES; ++w)
    for (int l = 0; l < 64; ++l)
      for (int i = 0; i < C::MI; ++i)
        for (int j = 0; j < C::NI; ++j)
          for (int r = 0; r < 16; ++r) tiles[w].acc[l][i][j][r] = 0.0f;
  for (int w = 0; w < C::WAVES; ++w)
    for (int l = 0; l < 64; ++l) {
      g_fill_lane = l;
      if (la[w]) fill_prologue<C, MX, B_KN, true, GK>(cps[w][l], nk, w, smem);
      else fill_prologue<C, MX, B_KN, false, GK>(cps[w][l], nk, w, smem);
    }
  for (int w = 0; w < C::WAVES; ++w)
    emu_wave_step<C, MX, B_KN, GK>(tiles[w], nm[w], smem, nk, w / C::WGN, w % C::WGN, -1);
  for (int k = 0; k < nk; ++k) {
    for (int w = 0; w < C::WAVES; ++w)
      emu_wave_step<C, MX, B_KN, GK>(tiles[w], nm[w], smem, nk, w / C::WGN, w % C::WGN, k);
    if (k + 1 < nk)
      for (int w = 0; w < C::WAVES; ++w)
        for (int l = 0; l < 64; ++l) {
          g_fill_lane = l;
          if (la[w]) fill_step<C, MX, B_KN, true, GK>(cps[w][l], k, nk, w, smem);
          else fill_step<C, MX, B_KN, false, GK>(cps[w][l], k, nk, w, smem);
        }
  }
  // compare the accumulators with the reference
  double max_ref = 0.0, max_err = 0.0;
  int bad_row = -1, bad_col = -1;
  double bad_got = 0.0, bad_want = 0.0;
  for (int w = 0; w < C::WAVES; ++w) {
    const int wm = w / C::WGN, wn = w % C::WGN;
    if (nm[w] == 0) continue;
    for (int l = 0; l < 64; ++l)
      for (int i = 0; i < nm[w]; ++i)
        for (int j = 0; j < C::NI; ++j)
          for (int r = 0; r < 16; ++r) {
            const int row = wm * C::WM + i * 32 + 8 * (r / 4) + 4 * (l / 32) + r % 4;
            const int col = wn * C::WN + j * 32 + l % 32;
            const double want = value(row, col);
            if (std::isnan(want)) continue;
            const double got = tiles[w].acc[l][i][j][r];
            max_ref = std::max(max_ref, std::fabs(want));
            const double err = std::fabs(got - want);
            if (!(err <= max_err)) {
              max_err = err;
              bad_row = row;
              bad_col = col;
              bad_got = got;
              bad_want = want;
            }
          }
  }
  ++g_emulated_items;
  if (!(max_err <= 1e-4 * std::max(max_ref, 1e-30)))
    CHECK_FAIL("%s: emulated tile differs from the reference GEMM: max |err| %.3g (max |ref| %.3g) at tile "
               "(%d, %d): %.6g vs %.6g", what, max_err, max_ref, bad_row, bad_col, bad_got, bad_want);
  if (epilogue) epilogue(tiles.get());
}

// ------------------------------------------------------------------------------------------------
// The 4-wave kernel's epilogue on the emulated accumulators: the text of gemm_epilogue.inc, run by one
// host thread per kernel thread, with its workgroup barriers as host barriers (prep_sim.inc) and
// __expf as the host expf. The outputs it writes are then compared with the reference GEMM (stores)
// and, for SwiGLU, with the SwiGLU of the kernel's own fp32 accumulators: bf16 exactly, and the fused
// MX requant byte for byte against an independent quantiser.
static long g_epilogue_items = 0;

// e4m3 value of a code without its sign (0x7f is NaN)
static double e4m3_mag(int c) {
  const int e = (c >> 3) & 15, m = c & 7;
  return e == 0 ? std::ldexp((double)m, -9) : std::ldexp(1.0 + m / 8.0, e - 7);
}

// Deliberate faults of the epilogue replay (mut_epi_* scenarios; the comparisons must report them):
// 1 - exp off by 2^-10 relative; 2 - e4m3 conversion rounds toward zero; 3 - scale code one too high.
static int g_epi_mutation = 0;
static float epi_expf(float x) { return g_epi_mutation == 1 ? expf(x) * (1.0f + 1.0f / 1024) : expf(x); }
static uint32_t epi_e4m3(float v) {
  const uint32_t c = f32_to_e4m3(v);
  if (g_epi_mutation == 2 && (c & 0x7f) != 0 && e4m3_mag(c & 0x7f) > std::fabs((double)v)) return c - 1;
  return c;
}
static uint32_t epi_scale_code(float amax) { return mx_scale_code(amax) + (g_epi_mutation == 3 ? 1 : 0); }

template <class C, int EPI, class Tile>
static void epi_thread(const GGParams& p, const Tile* tiles, const ItemCtx& ctx, uint8_t* smem,
                       prep_sim::Barrier* bar, int tid) {
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int nt = ctx.nt, split = ctx.split, half = ctx.half, rows_valid = ctx.rows_valid;
  const int64_t tile_row0 = ctx.tile_row0;
  v16f acc[C::MI][C::NI];
  for (int i = 0; i < C::MI; ++i)
    for (int j = 0; j < C::NI; ++j) acc[i][j] = tiles[wave].acc[lane][i][j];
  (void)tid, (void)split, (void)half, (void)wm, (void)wn;
#define __syncthreads() bar->wait()
#define __builtin_amdgcn_sched_barrier(x) ((void)0)
#define __expf(x) epi_expf(x)
#define f32_to_e4m3(v) epi_e4m3(v)
#define mx_scale_code(a) epi_scale_code(a)
#include "../../hyper_multicore_amd/csrc/gemm_epilogue.inc"
#undef __syncthreads
#undef __builtin_amdgcn_sched_barrier
#undef __expf
#undef f32_to_e4m3
#undef mx_scale_code
}

// One 32-value block: e8m0 code = the smallest e with amax <= 448 * 2^e (searched), each element the
// nearest e4m3 value of v / 2^e (searched over the codes, ties to the even code).
static void mx_block_ref(const float* v, uint8_t* q, uint8_t* code) {
  double amax = 0.0;
  for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs((double)v[i]));
  int e = -127;
  if (amax > 0.0)
    while (e < 127 && amax > 448.0 * std::ldexp(1.0, e)) ++e;
  *code = (uint8_t)(e + 127);
  for (int i = 0; i < 32; ++i) {
    const double s = std::fabs((double)v[i]) / std::ldexp(1.0, e);
    int best = 0;
    double bd = INFINITY;
    for (int c = 0; c < 0x7f; ++c) {
      const double d = std::fabs(e4m3_mag(c) - s);
      if (d < bd || (d == bd && (c & 1) == 0)) {
        bd = d;
        best = c;
      }
    }
    q[i] = (uint8_t)(best | (std::signbit(v[i]) ? 0x80 : 0));
  }
}

// n host threads kept for the epilogue replays (creating a workgroup's threads per item dominated the
// replay's time): run(f) calls f(t) on thread t = 0..n-1 and returns when all have returned.
struct EpiPool {
  explicit EpiPool(int n) : n_(n), start_(n + 1), done_(n + 1) {
    for (int t = 0; t < n; ++t)
      th_.emplace_back([this, t] {
        for (;;) {
          start_.wait();
          if (quit_) return;
          job_(t);
          done_.wait();
        }
      });
  }
  void run(const std::function<void(int)>& f) {
    job_ = f;
    start_.wait();
    done_.wait();
  }
  ~EpiPool() {
    quit_ = true;
    start_.wait();
    for (auto& x : th_) x.join();
  }
  int n_;
  prep_sim::Barrier start_, done_;
  std::function<void(int)> job_;
  bool quit_ = false;
  std::vector<std::thread> th_;
};

static EpiPool& epi_pool(int n) {
  static std::map<int, std::unique_ptr<EpiPool>> pools;
  auto& p = pools[n];
  if (!p) p.reset(new EpiPool(n));
  return *p;
}

template <class C, int EPI, class Tile>
static void emu_epilogue(const GGParams& p, const Tile* tiles, const ItemCtx& ctx,
                         const std::function<double(int, int)>& value) {
  constexpr bool SWIGLU = (EPI == EPI_SWIGLU_BF16 || EPI == EPI_SWIGLU_MX || EPI == EPI_SWIGLU_BF16_NUM);
  std::vector<uint8_t> lds(C::TOTAL, 0xa5);  // staging starts with garbage
  {
    prep_sim::Barrier bar(C::THREADS);
    epi_pool(C::THREADS).run([&](int t) { epi_thread<C, EPI>(p, tiles, ctx, lds.data(), &bar, t); });
  }
  ++g_epilogue_items;
  // the kernel's fp32 accumulator of tile element (row, col)
  auto acc_at = [&](int row, int col) -> float {
    const int wave = (row / C::WM) * C::WGN + col / C::WN;
    const int i = (row % C::WM) / 32, rr = row % 32, j = (col % C::WN) / 32;
    const int lane = 32 * ((rr >> 2) & 1) + col % 32, r = 4 * (rr >> 3) + (rr & 3);
    return tiles[wave].acc[lane][i][j][r];
  };
  double max_ref = 0.0;
  for (int row = 0; row < ctx.rows_valid; ++row)
    for (int c = 0; c < C::BN; ++c) {
      const double v = value(row, c);
      if (!std::isnan(v)) max_ref = std::max(max_ref, std::fabs(v));
    }
  long bad = 0;
  auto fail = [&](const char* what, int row, int col, double got, double want) {
    if (bad++ < 4)
      CHECK_FAIL("epilogue (%s) item g%d nt%d rows %lld+%d: (%d, %d) %.6g vs %.6g", what, ctx.g, ctx.nt,
                 (long long)ctx.tile_row0, ctx.rows_valid, row, col, got, want);
  };
  if (EPI == EPI_STORE_F32 || EPI == EPI_STORE_BF16) {
    for (int row = 0; row < ctx.rows_valid; ++row)
      for (int c = 0; c < C::BN; ++c) {
        const double want = value(row, c);
        if (std::isnan(want)) continue;
        const int64_t routed = ctx.tile_row0 + row;
        double got;
        if (EPI == EPI_STORE_F32) {
          const int64_t orow = p.c_row_index ? p.c_row_index[routed] : routed;
          got = ((const float*)p.C)[ctx.split * p.c_split_stride + orow * p.ldc + (int64_t)ctx.nt * C::BN + c];
          if (got != acc_at(row, c)) fail("fp32 store", row, c, got, acc_at(row, c));
        } else {
          got = bf16f(((const uint16_t*)p.C)[routed * p.ldc + (int64_t)ctx.nt * C::BN + c]);
          if (f32_to_bf16(acc_at(row, c)) != ((const uint16_t*)p.C)[routed * p.ldc + (int64_t)ctx.nt * C::BN + c])
            fail("bf16 store", row, c, got, acc_at(row, c));
        }
        if (!(std::fabs(got - want) <= std::ldexp(std::fabs(want), -8) + 2e-4 * max_ref))
          fail("store vs reference", row, c, got, want);
      }
    return;
  }
  if constexpr (SWIGLU) {
    constexpr int HW = C::WN / 2;
    const int ncol = C::BN / 2;
    std::vector<float> act(ncol);
    for (int row = 0; row < ctx.rows_valid; ++row) {
      const int64_t routed = ctx.tile_row0 + row;
      bool live[C::BN / 2];
      for (int j = 0; j < ncol; ++j) {
        const int gc = (j / HW) * C::WN + j % HW, uc = gc + HW;
        const double g_ref = value(row, gc), u_ref = value(row, uc);
        live[j] = !std::isnan(g_ref) && !std::isnan(u_ref) && (ctx.half < 0 || j / (ncol / 2) == ctx.half);
        act[j] = 0.0f;
        if (!live[j]) continue;
        // the SwiGLU of the kernel's accumulators (gemm_epilogue.inc's arithmetic)
        float gte = bf16_to_f32(f32_to_bf16(acc_at(row, gc)));
        float up = bf16_to_f32(f32_to_bf16(acc_at(row, uc)));
        float a;
        if (EPI == EPI_SWIGLU_BF16_NUM && p.swiglu_limit > 0.0f) {
          const float L = p.swiglu_limit;
          up = fminf(fmaxf(up, -L), L);
          if (p.swiglu_after_silu) a = fminf(gte / (1.0f + expf(-gte)), L) * up;
          else {
            const float gcl = fminf(gte, L);
            a = gcl / (1.0f + expf(-gcl)) * up;
          }
        } else {
          a = gte / (1.0f + expf(-gte)) * up;
        }
        act[j] = a;
        // and that of the reference GEMM (double), loosely: it pins the column pairing
        const double gr = bf16f(f32_to_bf16((float)g_ref)), ur = bf16f(f32_to_bf16((float)u_ref));
        double ar = gr / (1.0 + std::exp(-gr)) * ur;
        if (EPI == EPI_SWIGLU_BF16_NUM && p.swiglu_limit > 0.0f) {  // MegaMoeNumericsOptions clamp
          const double L = p.swiglu_limit, uc = std::min(std::max(ur, -L), L);
          if (p.swiglu_after_silu) ar = std::min(gr / (1.0 + std::exp(-gr)), L) * uc;
          else ar = std::min(gr, L) / (1.0 + std::exp(-std::min(gr, L))) * uc;
        }
        if (!(std::fabs(a - ar) <= 2e-2 * std::fabs(ar) + 1e-3 * max_ref * max_ref)) fail("SwiGLU vs reference", row, j, a, ar);
      }
      if (EPI == EPI_SWIGLU_MX) {
        for (int blk = 0; blk < ncol / 32; ++blk) {
          if (!live[blk * 32]) continue;
          uint8_t q[32], code;
          mx_block_ref(&act[blk * 32], q, &code);
          const uint8_t* got = (const uint8_t*)p.C + routed * p.ldc + (int64_t)ctx.nt * ncol + blk * 32;
          const uint8_t gcode = p.c_scale[routed * p.c_scale_ld + ctx.nt * 4 + blk];
          if (gcode != code) fail("MX scale code", row, blk * 32, gcode, code);
          for (int i = 0; i < 32; ++i)
            if (got[i] != q[i]) fail("MX element", row, blk * 32 + i, got[i], q[i]);
        }
      } else {
        const uint16_t* out = (const uint16_t*)p.C + routed * p.ldc + (int64_t)ctx.nt * ncol;
        for (int j = 0; j < ncol; ++j) {
          if (!live[j]) continue;
          float v = act[j];
          if (EPI == EPI_SWIGLU_BF16_NUM && p.row_prob != nullptr)
            v = bf16_to_f32(f32_to_bf16(v)) * p.row_prob[p.a_row_index[routed]];
          if (out[j] != f32_to_bf16(v)) fail("bf16 SwiGLU", row, j, bf16f(out[j]), v);
        }
      }
    }
  }
}

// Forward work items that ran as a column half of their tile
static long g_half_items = 0;

// ------------------------------------------------------------------------------------------------
// Forward grouped GEMM: all work items, waves and lanes
template <class C, bool MX, bool B_KN, int EPI>
static int sim_forward(const GGParams& p) {
  constexpr bool SWIGLU = (EPI == EPI_SWIGLU_BF16 || EPI == EPI_SWIGLU_MX || EPI == EPI_SWIGLU_BF16_NUM);
  constexpr int ESIZE = MX ? 1 : 2;
  ++g_gemms;
  // the kernel's own checks on the parameters it assumes
  if (!find_alloc(p.tile_prefix, (size_t)(p.G + 1) * 4)) CHECK_FAIL("tile prefix outside its buffer");
  if (!find_alloc(p.group_list, (size_t)p.G * 8)) CHECK_FAIL("group list outside its buffer");
  const int32_t* prefix = p.tile_prefix;
  // the two set-up lines of grouped_gemm_kernel
  const int splits = (EPI == EPI_STORE_F32 && p.k_splits > 1) ? p.k_splits : 1;
  const int items = prefix[p.G] * p.n_tiles;
  const int nk = p.K / splits * ESIZE / C::KB;  // stages per work item
  // the kernel's column halves of a partial last round, at launch_gg's grid on the stand-in's 256 CUs
  int tail_from = INT32_MAX;
  if (C::HALF_TAIL && EPI != EPI_STORE_F32 && EPI != EPI_STORE_BF16) {
    const int grid = (256 / 8) * 8 * C::WG_PER_CU;
    const int full = items / grid * grid;
    if (items > full && 2 * (items - full) <= grid) tail_from = full;
  }
  const int total = splits > 1 ? items * splits : (tail_from < items ? tail_from + 2 * (items - tail_from) : items);
  if (nk < 1) CHECK_FAIL("K = %d gives %d stages", p.K, nk);
  Layout lay;
  if (g_expect.set) {
    lay = {g_expect.A, g_expect.a_row_bytes, p.a_row_index, p.a_row_div, g_expect.a_scale, g_expect.a_scale_ld,
         g_expect.B, !B_KN, p.K, p.Ntot, ESIZE, g_expect.b_scale, g_expect.b_scale_ld};
  } else {
    lay = {p.A, p.lda_bytes, p.a_row_index, p.a_row_div, p.a_scale, p.a_scale_ld, p.B, !B_KN, p.K, p.Ntot, ESIZE,
         p.b_scale, p.b_scale_ld};
  }
  auto cps = std::make_unique<CopyPlan<C>[][64]>(C::WAVES);
  for (int L_item = 0; L_item < total; ++L_item) {
    ItemCtx ctx;
    std::vector<Rec> rec;
    std::vector<Wait> waits;
    bool first = true;
    bool las[C::WAVES];
    for (int wave = 0; wave < C::WAVES; ++wave)
      for (int lane = 0; lane < 64; ++lane) {
        const int L = L_item;
#include "../../hyper_multicore_amd/csrc/gemm_item_fwd.inc"
        cps[wave][lane] = cp;
        (void)mt;
        if (first) {
          first = false;
          ++g_items;
          ctx.g = g;
          ctx.nt = nt;
          ctx.split = split;
          ctx.nk = nk;
          ctx.half = half;
          if (half >= 0) ++g_half_items;
          ctx.tile_row0 = tile_row0;
          ctx.rows_valid = rows_valid;
          ctx.cov[R_A].assign((size_t)nk * C::A_BYTES, 0);
          ctx.cov[R_B].assign((size_t)nk * C::B_BYTES, 0);
          ctx.cov[R_BS].assign((size_t)nk * C::BS_BYTES, 0);
          const int ng = (nk + 7) / 8 + 1;
          ctx.cov[R_AS].assign((size_t)ng * C::AS_SLOT, 0);
          ctx.cov[R_BSR].assign((size_t)ng * C::BSR_SLOT, 0);
          if (rows_valid < 1 || rows_valid > C::BM) CHECK_FAIL("item %d: %d valid rows", L_item, rows_valid);
          if (g < 0 || g >= p.G || nt < 0 || nt >= p.n_tiles) CHECK_FAIL("item %d decodes to group %d n-tile %d", L_item, g, nt);
          // epilogue output range of this tile
          const int64_t r0 = tile_row0, r1 = tile_row0 + rows_valid - 1;
          if (EPI == EPI_STORE_BF16) {
            const int64_t cols = std::min<int64_t>(C::BN, p.N - (int64_t)nt * C::BN);
            check_range(p.C, (r0 * p.ldc + (int64_t)nt * C::BN) * 2, (r1 * p.ldc + (int64_t)nt * C::BN + cols) * 2,
                        "bf16 epilogue");
          } else if (EPI == EPI_STORE_F32) {
            const int64_t cols = std::min<int64_t>(C::BN, p.N - (int64_t)nt * C::BN);
            for (int64_t r = r0; r <= r1; ++r) {
              const int64_t orow = p.c_row_index ? p.c_row_index[r] : r;
              const int64_t at = split * p.c_split_stride + orow * p.ldc + (int64_t)nt * C::BN;
              check_range(p.C, at * 4, (at + cols) * 4, "fp32 epilogue");
            }
          } else if (EPI == EPI_SWIGLU_MX) {
            check_range(p.C, r0 * p.ldc + (int64_t)nt * (C::BN / 2), r1 * p.ldc + (int64_t)nt * (C::BN / 2) + C::BN / 2,
                        "MX SwiGLU epilogue");
            check_range(p.c_scale, r0 * p.c_scale_ld + nt * 4, r1 * p.c_scale_ld + nt * 4 + 4, "MX SwiGLU scales");
            if ((int64_t)nt * (C::BN / 2) + C::BN / 2 > p.N) CHECK_FAIL("MX SwiGLU tile past N = %d", p.N);
          } else {
            check_range(p.C, (r0 * p.ldc + (int64_t)nt * (C::BN / 2)) * 2,
                        (r1 * p.ldc + (int64_t)nt * (C::BN / 2) + C::BN / 2) * 2, "SwiGLU epilogue");
            if ((int64_t)nt * (C::BN / 2) + C::BN / 2 > p.N) CHECK_FAIL("SwiGLU tile past N = %d", p.N);
            if (EPI == EPI_SWIGLU_BF16_NUM && p.row_prob != nullptr)
              for (int64_t r = r0; r <= r1; ++r)
                if (!find_alloc(p.row_prob + p.a_row_index[r], 4)) CHECK_FAIL("row probability of row %lld", (long long)r);
          }
        }
        const bool la = wave_copies_a<C>(wave, rows_valid);
        las[wave] = la;
        rec.clear();
        waits.clear();
        if (la) record_schedule<C, MX, B_KN, true, false>(cp, nk, wave, rec, waits);
        else record_schedule<C, MX, B_KN, false, false>(cp, nk, wave, rec, waits);
        check_lane<C, MX, B_KN, SWIGLU, false>(p, lay, ctx, wave, lane, la, rec, waits);
      }
    check_coverage<C, MX, B_KN, false>(ctx);
    if (g_emulate) {
      int nms[C::WAVES];
      for (int w = 0; w < C::WAVES; ++w) {  // the kernel's subtile count per wave
        const int rows_w = ctx.rows_valid - (w / C::WGN) * C::WM;
        nms[w] = (C::MI >= 4 && rows_w > 64) ? 4 : ((C::MI >= 2 && rows_w > 32) ? 2 : (rows_w >= 1 ? 1 : 0));
        if (ctx.half >= 0 && ((w % C::WGN) >> 1) != ctx.half) nms[w] = 0;  // the other half's waves
      }
      const int Kper = p.K / splits;
      auto value = [&](int row, int col) -> double {
        int64_t wc;
        if (ctx.half >= 0 && col / (C::BN / 2) != ctx.half) return NAN;
        if (row >= ctx.rows_valid || !tile_weight_col<C>(col, ctx.nt, p.N, SWIGLU, p.gate_up_interleaved, &wc)) return NAN;
        const int64_t r = ctx.tile_row0 + row;
        const int64_t sr = p.a_row_index ? p.a_row_index[r] / p.a_row_div : r;
        double sum = 0.0;
        for (int k = ctx.split * Kper; k < (ctx.split + 1) * Kper; ++k) {
          double av, bv;
          if (!MX) {
            uint16_t a16, b16;
            memcpy(&a16, p.A + sr * p.lda_bytes + 2 * (int64_t)k, 2);
            const uint8_t* bp = p.B + (int64_t)ctx.g * p.b_group_stride +
                                (B_KN ? (int64_t)k * p.b_row_bytes + wc * 2 : wc * p.b_row_bytes + 2 * (int64_t)k);
            memcpy(&b16, bp, 2);
            av = bf16f(a16);
            bv = bf16f(b16);
          } else {
            av = e4m3f(p.A[sr * p.lda_bytes + k]) * e8m0f(p.a_scale[sr * p.a_scale_ld + k / 32]);
            const uint8_t* gb = p.B + (int64_t)ctx.g * p.b_group_stride;
            if (B_KN) {
              bv = e4m3f(gb[(int64_t)k * p.b_row_bytes + wc]) *
                   e8m0f(p.b_scale[(int64_t)ctx.g * p.b_scale_group_stride + ((k / 64) * (int64_t)p.Ntot + wc) * 2 +
                                   ((k / 32) & 1)]);
            } else {
              bv = e4m3f(gb[wc * p.b_row_bytes + k]) *
                   e8m0f(p.b_scale[((int64_t)ctx.g * p.Ntot + wc) * p.b_scale_ld + k / 32]);
            }
          }
          sum += av * bv;
        }
        return sum;
      };
      emulate_item<C, MX, B_KN, false>(*reinterpret_cast<const CopyPlan<C>(*)[C::WAVES][64]>(cps.get()), las, nms, nk,
                                        value, "forward item", [&](const EmuWaveTile<C, MX, B_KN, false>* tiles) {
                                          emu_epilogue<C, EPI>(p, tiles, ctx, value);
                                        });
    }
  }
  return MI355MOE_OK;
}

template <class C, bool MX, int EPI>
static int sim_wgrad(const GGParams& p) {
  ++g_gemms;
  if (!find_alloc(p.group_list, (size_t)p.G * 8)) CHECK_FAIL("group list outside its buffer");
  const int per_g = p.m_tiles * p.n_tiles;
  const int total = p.G * per_g;
  constexpr int ES = MX ? 1 : 2;
  Layout Lo = {p.A, p.lda_bytes, nullptr, 1, nullptr, 0, p.B, false, 0, 0, ES, nullptr, 0};
  if (g_expect.set) {
    Lo.A = g_expect.A;
    Lo.a_row_bytes = g_expect.a_row_bytes;
    Lo.B = g_expect.B;
  }
  Lo.Ntot = p.b_row_bytes / ES;  // B rows hold N elements (grouped-K: row stride of the routed rows)
  if (g_expect.set) Lo.Ntot = p.N;
  auto cps = std::make_unique<CopyPlan<C>[][64]>(C::WAVES);
  for (int L_item = 0; L_item < total; ++L_item) {
    ItemCtx ctx;
    std::vector<Rec> rec;
    std::vector<Wait> waits;
    bool first = true;
    for (int wave = 0; wave < C::WAVES; ++wave)
      for (int lane = 0; lane < 64; ++lane) {
        const int L = L_item;
#include "../../hyper_multicore_amd/csrc/gemm_item_wgrad.inc"
        cps[wave][lane] = cp;
        (void)mt;
        if (first) {
          first = false;
          ++g_items;
          ctx.g = g;
          ctx.nt = nt;
          ctx.split = 0;
          ctx.nk = nk;
          ctx.k0 = k0;
          ctx.kend = kend;
          ctx.m0 = m0;
          ctx.rows_valid = rows_valid;
          ctx.cov[R_A].assign((size_t)std::max(nk, 0) * C::A_BYTES, 0);
          ctx.cov[R_B].assign((size_t)std::max(nk, 0) * C::B_BYTES, 0);
          ctx.cov[R_BS].assign((size_t)std::max(nk, 0) * C::BS_BYTES, 0);
          ctx.cov[R_ASS].assign((size_t)std::max(nk, 0) * C::BS_BYTES, 0);
          const int64_t cols = std::min<int64_t>(C::BN, p.N - (int64_t)nt * C::BN);
          const int esz = EPI == EPI_STORE_F32 ? 4 : 2;
          const int64_t at0 = (int64_t)g * p.c_group_stride + (int64_t)m0 * p.ldc + (int64_t)nt * C::BN;
          const int64_t at1 = (int64_t)g * p.c_group_stride + (int64_t)(m0 + rows_valid - 1) * p.ldc + (int64_t)nt * C::BN + cols;
          check_range(p.C, at0 * esz, at1 * esz, "weight-gradient epilogue");
        }
        if (nk <= 0) continue;
        rec.clear();
        waits.clear();
        record_schedule<C, MX, true, true, true>(cp, nk, wave, rec, waits);
        check_lane<C, MX, true, false, true>(p, Lo, ctx, wave, lane, true, rec, waits);
      }
    if (ctx.nk > 0) check_coverage<C, MX, true, true>(ctx);
    if (g_emulate && ctx.nk > 0) {
      bool las[C::WAVES];
      int nms[C::WAVES];
      for (int w = 0; w < C::WAVES; ++w) {
        las[w] = true;
        const int rows_w = ctx.rows_valid - (w / C::WGN) * C::WM;
        nms[w] = (C::MI >= 4 && rows_w > 64) ? 4 : ((C::MI >= 2 && rows_w > 32) ? 2 : (rows_w >= 1 ? 1 : 0));
      }
      auto value = [&](int row, int col) -> double {
        const int64_t m = (int64_t)ctx.m0 + row, n = (int64_t)ctx.nt * C::BN + col;
        if (row >= ctx.rows_valid || n >= p.N) return NAN;
        double sum = 0.0;
        for (int64_t r = ctx.k0; r < ctx.kend; ++r) {
          double av, bv;
          if (!MX) {
            uint16_t a16, b16;
            memcpy(&a16, p.A + r * p.lda_bytes + 2 * m, 2);
            memcpy(&b16, p.B + r * p.b_row_bytes + 2 * n, 2);
            av = bf16f(a16);
            bv = bf16f(b16);
          } else {
            const int64_t grp = ctx.k0 / 64 + ctx.g + (r - ctx.k0) / 64, half = ((r - ctx.k0) / 32) & 1;
            av = e4m3f(p.A[r * p.lda_bytes + m]) * e8m0f(p.a_scale[(grp * p.m_rows + m) * 2 + half]);
            bv = e4m3f(p.B[r * p.b_row_bytes + n]) * e8m0f(p.b_scale[(grp * p.N + n) * 2 + half]);
          }
          sum += av * bv;
        }
        return sum;
      };
      emulate_item<C, MX, true, true>(*reinterpret_cast<const CopyPlan<C>(*)[C::WAVES][64]>(cps.get()), las, nms,
                                       ctx.nk, value, "grouped-K item");
    }
  }
  return MI355MOE_OK;
}


// The grouped GEMM entry points the host code calls, run on the host
template <class C>
static int sim_dispatch(const GGParams& p, bool mx, bool b_kn, int epi) {
  if (!mx) {
    if (!b_kn) {
      switch (epi) {
        case EPI_STORE_BF16: return sim_forward<C, false, false, EPI_STORE_BF16>(p);
        case EPI_STORE_F32: return sim_forward<C, false, false, EPI_STORE_F32>(p);
        case EPI_SWIGLU_BF16: return sim_forward<C, false, false, EPI_SWIGLU_BF16>(p);
        case EPI_SWIGLU_BF16_NUM: return sim_forward<C, false, false, EPI_SWIGLU_BF16_NUM>(p);
      }
    } else {
      switch (epi) {
        case EPI_STORE_BF16: return sim_forward<C, false, true, EPI_STORE_BF16>(p);
        case EPI_SWIGLU_BF16: return sim_forward<C, false, true, EPI_SWIGLU_BF16>(p);
        case EPI_SWIGLU_BF16_NUM: return sim_forward<C, false, true, EPI_SWIGLU_BF16_NUM>(p);
      }
    }
  } else if constexpr (C::AS_N == 0) {
    return MI355MOE_EUNSUPPORTED;
  } else if (!b_kn) {
    if constexpr (C::BSR_N == 0) {
      return MI355MOE_EUNSUPPORTED;
    } else {
      switch (epi) {
        case EPI_STORE_BF16: return sim_forward<C, true, false, EPI_STORE_BF16>(p);
        case EPI_SWIGLU_MX: return sim_forward<C, true, false, EPI_SWIGLU_MX>(p);
      }
    }
  } else {
    switch (epi) {
      case EPI_STORE_BF16: return sim_forward<C, true, true, EPI_STORE_BF16>(p);
      case EPI_SWIGLU_MX: return sim_forward<C, true, true, EPI_SWIGLU_MX>(p);
    }
  }
  CHECK_FAIL("no kernel for mx=%d b_kn=%d epilogue %d", mx, b_kn, epi);
  return MI355MOE_EUNSUPPORTED;
}

// ------------------------------------------------------------------------------------------------
// The 8-wave configuration (gemm_pp.hip): replayed when a scenario routes GEMMs to it as the library
// does (g_pp_route); otherwise the library's forward is steered onto the 4-wave and decode kernels.
static bool g_pp_route = false;
#include "pp_sim.inc"

// Library internals replaced by the simulation (same signatures as gemm.h). gemm_pp.hip's own
// mi355_gg_pp_usable is linked under the name below.
bool mi355_gg_pp_usable_lib(int variant, bool mx, bool b_kn, int64_t K, int G, int64_t a_bytes, int64_t b_group_stride);
bool mi355_gg_pp_usable(int variant, bool mx, bool b_kn, int64_t K, int G, int64_t a_bytes, int64_t b_group_stride) {
  return g_pp_route && mi355_gg_pp_usable_lib(variant, mx, b_kn, K, G, a_bytes, b_group_stride);
}

int mi355_grouped_gemm(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t, bool small) {
  // the dispatcher's choice of the numerics epilogue (gemm.hip, mi355_grouped_gemm)
  if (epi == EPI_SWIGLU_BF16_NUM) return MI355MOE_EINVAL;
  if (epi == EPI_SWIGLU_BF16 && (p.swiglu_limit > 0.0f || p.row_prob != nullptr)) epi = EPI_SWIGLU_BF16_NUM;
  if (g_force_big) small = false;
  if (small) return sim_dispatch<GGSmall>(p, mx, b_kn, epi);
  // the 8-wave configuration first (gemm.hip's order); the 4-wave kernels for what it does not take
  if (g_pp_route && (p.variant == MI355_GG_VARIANT_DEFAULT || p.variant == MI355_GG_VARIANT_PP)) {
    const int rc = mi355_grouped_gemm_pp(p, mx, b_kn, epi, nullptr);
    if (rc != MI355MOE_EUNSUPPORTED) return rc;
  }
  if (p.a_scale_stage_stride != 0 || p.c_scale_stage_stride != 0) return MI355MOE_EUNSUPPORTED;
  return sim_dispatch<GGBig>(p, mx, b_kn, epi);
}
int mi355_grouped_gemm_wgrad(const GGParams& p, int epi, hipStream_t, bool mx) {
  // the checks of gemm_wgrad.hip's mi355_grouped_gemm_wgrad
  const int align = mx ? 16 : 8;
  if (p.m_rows % align || p.N % align || p.m_tiles != (p.m_rows + GGBig::BM - 1) / GGBig::BM ||
      p.n_tiles != (p.N + GGBig::BN - 1) / GGBig::BN || p.zero_row == nullptr)
    return MI355MOE_EINVAL;
  if (mx && (p.a_scale == nullptr || p.b_scale == nullptr)) return MI355MOE_EINVAL;
  const Alloc* z = alloc_of(p.zero_row);
  const int64_t need = (int64_t)std::max(p.m_rows, p.N) * (mx ? 1 : 2);
  if (!z || p.zero_row + need > z->p + z->n) CHECK_FAIL("zero row shorter than %lld bytes", (long long)need);
  if (epi == EPI_STORE_F32) return mx ? sim_wgrad<GGBig, true, EPI_STORE_F32>(p) : sim_wgrad<GGBig, false, EPI_STORE_F32>(p);
  if (epi == EPI_STORE_BF16) return mx ? sim_wgrad<GGBig, true, EPI_STORE_BF16>(p) : sim_wgrad<GGBig, false, EPI_STORE_BF16>(p);
  return MI355MOE_EUNSUPPORTED;
}

// ------------------------------------------------------------------------------------------------
// Scenarios: C-ABI calls with host buffers sized from the shapes the header documents
static std::mt19937_64 g_rng(20261201);

// Random operands for the emulated scenarios: bf16 in +-[0.5, 2), e4m3 codes except the NaN code,
// e8m0 scale codes near 2^0.
static void fill_bf16(uint8_t* p, size_t count) {
  std::uniform_real_distribution<float> u(0.5f, 2.0f);
  for (size_t i = 0; i < count; ++i) {
    float v = u(g_rng) * ((g_rng() & 1) ? -1.0f : 1.0f);
    uint32_t b;
    memcpy(&b, &v, 4);
    const uint16_t h = (uint16_t)(b >> 16);
    memcpy(p + 2 * i, &h, 2);
  }
}
static void fill_e4m3(uint8_t* p, size_t count) {
  for (size_t i = 0; i < count; ++i) {
    uint8_t v = (uint8_t)(g_rng() & 0xff);
    if ((v & 0x7f) == 0x7f) v ^= 1;
    p[i] = v;
  }
}
static void fill_codes(uint8_t* p, size_t count) {
  for (size_t i = 0; i < count; ++i) p[i] = (uint8_t)(120 + g_rng() % 14);
}

static std::vector<int64_t> cumsum(const std::vector<int>& counts) {
  std::vector<int64_t> gl(counts.size());
  int64_t a = 0;
  for (size_t i = 0; i < counts.size(); ++i) gl[i] = a += counts[i];
  return gl;
}

static int expect_rc(int rc, int want, const char* what) {
  if (rc != want) CHECK_FAIL("%s returned %d (expected %d)", what, rc, want);
  return rc;
}

static void gemm_bf16(std::vector<int> counts, int K, int N, int layout, bool noalloc = false) {
  const int G = (int)counts.size();
  const auto glv = cumsum(counts);
  const int64_t rows = glv.back();
  uint8_t* x = mk("x", (size_t)rows * K * 2);
  uint8_t* w = mk("w", (size_t)G * K * N * 2);
  if (g_emulate) {
    fill_bf16(x, (size_t)rows * K);
    fill_bf16(w, (size_t)G * K * N);
  }
  uint8_t* out = mk("out", (size_t)rows * N * 2);
  int64_t* gl = (int64_t*)mk("group_list", G * 8);
  memcpy(gl, glv.data(), G * 8);
  const size_t wsz = mi355moe_grouped_gemm_workspace_size(G);
  uint8_t* ws = mk("workspace", wsz);
  g_expect = Expect();
  g_expect.set = true;
  g_expect.A = x;
  g_expect.a_row_bytes = (int64_t)K * 2;
  g_expect.B = w;
  if (noalloc)
    expect_rc(mi355moe_grouped_gemm_bf16_noalloc((const uint16_t*)x, rows, K, (const uint16_t*)w, layout, G, N, gl,
                                                 (uint16_t*)out, g_variant, nullptr),
              0, "grouped_gemm_bf16_noalloc");
  else
    expect_rc(mi355moe_grouped_gemm_bf16((const uint16_t*)x, rows, K, (const uint16_t*)w, layout, G, N, gl,
                                         (uint16_t*)out, g_variant, ws, wsz, nullptr),
              0, "grouped_gemm_bf16");
  g_expect = Expect();
}

static void gemm_mx(std::vector<int> counts, int K, int N, int layout) {
  const int G = (int)counts.size();
  const auto glv = cumsum(counts);
  const int64_t rows = glv.back();
  uint8_t* xq = mk("xq", (size_t)rows * K);
  uint8_t* xs = mk("x_scale", (size_t)rows * (K / 32));
  uint8_t* wd = mk("w_data", (size_t)G * K * N);
  const bool eoi = layout == MI355MOE_LAYOUT_EOI;
  const int64_t sld = mi355moe_mx_weight_scale_ld(K);
  uint8_t* wsc = eoi ? mk("w_scale_eoi", (size_t)G * N * sld) : mk("col_scale", (size_t)G * (K / 64) * N * 2);
  if (g_emulate) {
    fill_e4m3(xq, (size_t)rows * K);
    fill_codes(xs, (size_t)rows * (K / 32));
    fill_e4m3(wd, (size_t)G * K * N);
    fill_codes(wsc, eoi ? (size_t)G * N * sld : (size_t)G * (K / 64) * N * 2);
  }
  uint8_t* out = mk("out", (size_t)rows * N * 2);
  int64_t* gl = (int64_t*)mk("group_list", G * 8);
  memcpy(gl, glv.data(), G * 8);
  const size_t wsz = mi355moe_grouped_gemm_workspace_size(G);
  uint8_t* ws = mk("workspace", wsz);
  g_expect = Expect();
  g_expect.set = true;
  g_expect.A = xq;
  g_expect.a_row_bytes = K;
  g_expect.a_scale = xs;
  g_expect.a_scale_ld = K / 32;
  g_expect.B = wd;
  g_expect.b_scale = wsc;
  g_expect.b_scale_ld = sld;
  expect_rc(mi355moe_grouped_gemm_mxfp8(xq, xs, rows, K, wd, wsc, layout, G, N, gl, (uint16_t*)out, g_variant, ws, wsz, nullptr),
            0, "grouped_gemm_mxfp8");
  g_expect = Expect();
}

// Routed ids for T tokens: distinct experts per token, drawn from a skewed popularity.
static std::vector<int64_t> route_ids(int64_t T, int K, int E, double skew) {
  std::vector<double> wgt(E);
  for (int e = 0; e < E; ++e) wgt[e] = 1.0 / std::pow(1.0 + e, skew);
  std::vector<int> perm(E);
  for (int e = 0; e < E; ++e) perm[e] = e;
  std::shuffle(perm.begin(), perm.end(), g_rng);
  std::vector<int64_t> ids((size_t)T * K);
  for (int64_t t = 0; t < T; ++t) {
    std::vector<double> w = wgt;
    for (int k = 0; k < K; ++k) {
      std::discrete_distribution<int> d(w.begin(), w.end());
      const int e = d(g_rng);
      w[e] = 0.0;
      ids[(size_t)t * K + k] = perm[e];
    }
  }
  return ids;
}

// The 8-wave configuration on GGParams built here as the forward builds them (api.hip): routed rows
// gathered from `fanout` slots per token, MX activation scales as stage-major code planes by routed
// row, SwiGLU on [gate | up] weight columns (optionally gate/up interleaved). With g_emulate the
// outputs are compared with the reference; for the MX SwiGLU GEMM the fp32 epilogue (the library's)
// and the MXFP8 epilogue run on the same operands and the latter must equal the MX quantisation of
// the former, byte for byte.
static void pp_gemm(std::vector<int> counts, int K, int N, bool mx, bool b_kn, bool swiglu, int gu) {
  const int G = (int)counts.size(), esize = mx ? 1 : 2;
  const auto glv = cumsum(counts);
  const int64_t R = glv.back();
  const int fanout = 2;
  const int64_t T = (R + fanout - 1) / fanout;
  const int Ntot = swiglu ? 2 * N : N;
  uint8_t* A = mk("pp_A", (size_t)T * K * esize);
  int32_t* gather = (int32_t*)mk("pp_gather", (size_t)R * 4);
  {
    std::vector<int32_t> slots(T * fanout);
    for (size_t i = 0; i < slots.size(); ++i) slots[i] = (int32_t)i;
    std::shuffle(slots.begin(), slots.end(), g_rng);
    for (int64_t r = 0; r < R; ++r) gather[r] = slots[r];
  }
  uint8_t* B = mk("pp_B", (size_t)G * K * Ntot * esize);
  const int64_t planes = (int64_t)(K / 128) * 4 * R + 512;
  uint8_t* as = mx ? mk("pp_A_scale_planes", (size_t)planes) : nullptr;
  uint8_t* bs = mx ? mk("pp_col_scale", (size_t)G * (K / 64) * Ntot * 2) : nullptr;
  int64_t* gl = (int64_t*)mk("pp_group_list", G * 8);
  memcpy(gl, glv.data(), G * 8);
  if (g_emulate) {
    if (mx) {
      fill_e4m3(A, (size_t)T * K);
      fill_e4m3(B, (size_t)G * K * Ntot);
      fill_codes(as, (size_t)planes);
      fill_codes(bs, (size_t)G * (K / 64) * Ntot * 2);
    } else {
      fill_bf16(A, (size_t)T * K);
      fill_bf16(B, (size_t)G * K * Ntot);
    }
  }
  GGParams p = {};
  p.A = A;
  p.lda_bytes = (int64_t)K * esize;
  p.a_bytes = T * K * esize;
  p.a_row_index = gather;
  p.a_row_div = fanout;
  p.B = B;
  p.b_group_stride = (int64_t)K * Ntot * esize;
  p.b_row_bytes = b_kn ? (int64_t)Ntot * esize : (int64_t)K * esize;
  p.K = K;
  p.N = N;
  p.Ntot = Ntot;
  p.n_tiles = swiglu ? N / 128 : (N + 255) / 256;
  p.G = G;
  p.group_list = gl;
  p.rows_hint = R;
  p.gate_up_interleaved = gu;
  p.variant = MI355_GG_VARIANT_DEFAULT;
  if (mx) {
    p.a_scale = as;
    p.a_scale_stage_stride = R * 4;
    p.a_scale_routed = 1;
    p.b_scale = bs;
    p.b_scale_group_stride = (int64_t)(K / 64) * Ntot * 2;
  }
  const int epi = !swiglu ? EPI_STORE_BF16 : (mx ? EPI_SWIGLU_F32 : EPI_SWIGLU_BF16);
  p.C = mk("pp_C", (size_t)R * N * (epi == EPI_SWIGLU_F32 ? 4 : 2));
  p.ldc = N;
  expect_rc(mi355_grouped_gemm_pp(p, mx, b_kn, epi, nullptr), 0, "8-wave grouped GEMM");
  if (!(mx && swiglu)) return;
  // the MXFP8 SwiGLU epilogue on the same operands
  GGParams q = p;
  const int64_t cplanes = (int64_t)(N / 128) * 4 * R + 512;
  q.C = mk("pp_act_e4m3", (size_t)R * N);
  q.c_scale = mk("pp_act_planes", (size_t)cplanes);
  q.c_scale_stage_stride = R * 4;
  sim_pp<true, true, EPI_SWIGLU_MX, false, pp::SEL_ALL>(q);
  if (!g_emulate) return;
  const float* f = (const float*)p.C;
  const uint8_t* e = (const uint8_t*)q.C;
  long bad = 0;
  for (int64_t r = 0; r < R; ++r)
    for (int cb = 0; cb < N / 32; ++cb) {
      float amax = 0.0f;
      for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(f[r * N + cb * 32 + i]));
      const uint32_t code = mx_scale_code(amax);
      const uint8_t got_code = q.c_scale[(cb >> 2) * q.c_scale_stage_stride + (cb & 3) * (q.c_scale_stage_stride >> 2) + r];
      if (got_code != code && bad++ < 3) CHECK_FAIL("MX SwiGLU epilogue: scale code of row %lld block %d is %d, expected %u", (long long)r, cb, got_code, code);
      for (int i = 0; i < 32; ++i) {
        const uint8_t want = (uint8_t)(f32_to_e4m3(mx_apply_inv_scale(f[r * N + cb * 32 + i], code)) & 0xff);
        if (e[r * N + cb * 32 + i] != want && bad++ < 3)
          CHECK_FAIL("MX SwiGLU epilogue: element (%lld, %d) is 0x%02x, expected 0x%02x", (long long)r, cb * 32 + i,
                     e[r * N + cb * 32 + i], want);
      }
    }
  if (bad) CHECK_FAIL("MX SwiGLU epilogue: %ld bytes differ from the quantised fp32 epilogue", bad);
}

// runs f with replay fault `mutation` switched on: the scenario passes when the checks report it
static std::function<void()> pp_mutant(int mutation, std::function<void()> f) {
  return [mutation, f] {
    const long e0 = g_errors;
    g_pp_mutation = mutation;
    g_pp_copy_no = 0;
    f();
    g_pp_mutation = 0;
    const long found = g_errors - e0;
    g_errors = e0;
    if (found == 0) CHECK_FAIL("replay fault %d was not reported", mutation);
    else printf("replay fault %d reported (%ld findings)\n", mutation, found);
  };
}

// runs f with epilogue replay fault `mutation` switched on: the scenario passes when it is reported
static std::function<void()> epi_mutant(int mutation, std::function<void()> f) {
  return [mutation, f] {
    const long e0 = g_errors;
    g_epi_mutation = mutation;
    f();
    g_epi_mutation = 0;
    const long found = g_errors - e0;
    g_errors = e0;
    if (found == 0) CHECK_FAIL("epilogue fault %d was not reported", mutation);
    else printf("epilogue fault %d reported (%ld findings)\n", mutation, found);
  };
}

// runs f with the library's GEMMs routed to the 8-wave configuration as the library routes them;
// the scenario fails when no GEMM ran on it
static std::function<void()> pp_route(std::function<void()> f) {
  return [f] {
    const long before = g_pp_gemms;
    g_pp_route = true;
    f();
    g_pp_route = false;
    if (g_pp_gemms == before) CHECK_FAIL("no GEMM ran on the 8-wave configuration");
  };
}

static void moe_forward(int64_t T, int K, int E, int H, int I, int precision, int layout, double skew,
                        int numerics = 0, float limit = 0.0f) {
  const bool mx = precision == MI355MOE_PRECISION_MXFP8;
  const bool eoi = layout == MI355MOE_LAYOUT_EOI;
  const auto idv = route_ids(T, K, E, skew);
  uint8_t* hidden = mk("hidden", (size_t)T * H * 2);
  int64_t* ids = (int64_t*)mk("topk_ids", idv.size() * 8);
  memcpy(ids, idv.data(), idv.size() * 8);
  float* wts = (float*)mk("topk_weights", (size_t)T * K * 4, 0);
  const int esz = mx ? 1 : 2;
  uint8_t* w1 = mk("w1", (size_t)E * H * 2 * I * esz);
  uint8_t* w2 = mk("w2", (size_t)E * I * H * esz);
  uint8_t *s1 = nullptr, *s2 = nullptr;
  if (mx) {
    if (eoi) {
      s1 = mk("w1_scale_eoi", (size_t)E * 2 * I * mi355moe_mx_weight_scale_ld(H));
      s2 = mk("w2_scale_eoi", (size_t)E * H * mi355moe_mx_weight_scale_ld(I));
    } else {
      s1 = mk("w1_col_scale", (size_t)E * (H / 64) * 2 * I * 2);
      s2 = mk("w2_col_scale", (size_t)E * (I / 64) * H * 2);
    }
  }
  if (g_emulate) {  // operands of moderate size, so the emulated epilogues compare finite values
    std::uniform_real_distribution<float> pu(0.05f, 1.0f);
    for (int64_t i = 0; i < T * K; ++i) wts[i] = pu(g_rng);
    fill_bf16(hidden, (size_t)T * H);
    if (mx) {
      fill_e4m3(w1, (size_t)E * H * 2 * I);
      fill_e4m3(w2, (size_t)E * I * H);
      if (eoi) {
        fill_codes(s1, (size_t)E * 2 * I * mi355moe_mx_weight_scale_ld(H));
        fill_codes(s2, (size_t)E * H * mi355moe_mx_weight_scale_ld(I));
      } else {
        fill_codes(s1, (size_t)E * (H / 64) * 2 * I * 2);
        fill_codes(s2, (size_t)E * (I / 64) * H * 2);
      }
    } else {
      fill_bf16(w1, (size_t)E * H * 2 * I);
      fill_bf16(w2, (size_t)E * I * H);
    }
  }
  uint8_t* out = mk("out", (size_t)T * H * 2);
  MI355MoeForwardArgs a = {};
  a.hidden = (const uint16_t*)hidden;
  a.num_tokens = T;
  a.hidden_size = H;
  a.intermediate_size = I;
  a.num_experts = E;
  a.top_k = K;
  a.topk_ids = ids;
  a.ids_dtype = MI355MOE_IDS_INT64;
  a.precision = precision;
  a.topk_weights = wts;
  a.weight_layout = layout;
  a.numerics_flags = numerics;
  a.swiglu_limit = limit;
  a.gemm_variant = g_variant;
  a.w1 = w1;
  a.w2 = w2;
  a.w1_scale = s1;
  a.w2_scale = s2;
  a.out = (uint16_t*)out;
  const size_t wsz = mi355moe_moe_forward_workspace_size(&a);
  uint8_t* ws = mk("workspace", wsz);
  g_expect = Expect();  // internal operands: addressing from GGParams, bounds from the allocations
  expect_rc(mi355moe_moe_forward(&a, ws, wsz, nullptr), 0, "moe_forward");
}

static void moe_backward(int64_t T, int K, int E, int H, int I, int layout, int grad_dtype, double skew,
                         bool mx = false) {
  const auto idv = route_ids(T, K, E, skew);
  uint8_t* hidden = mk("hidden", (size_t)T * H * 2);
  int64_t* ids = (int64_t*)mk("topk_ids", idv.size() * 8);
  memcpy(ids, idv.data(), idv.size() * 8);
  float* wts = (float*)mk("topk_weights", (size_t)T * K * 4, 0);
  const int esz = mx ? 1 : 2;
  uint8_t* w1 = mk("w1", (size_t)E * H * 2 * I * esz);
  uint8_t* w2 = mk("w2", (size_t)E * I * H * esz);
  uint8_t* gout = mk("grad_out", (size_t)T * H * 2);
  uint8_t* gh = mk("grad_hidden", (size_t)T * H * 2);
  const int gsz = grad_dtype == MI355MOE_GRAD_FP32 ? 4 : 2;
  uint8_t* gw1 = mk("grad_w1", (size_t)E * H * 2 * I * gsz);
  uint8_t* gw2 = mk("grad_w2", (size_t)E * I * H * gsz);
  float* gp = (float*)mk("grad_topk_weights", (size_t)T * K * 4);
  MI355MoeBackwardArgs a = {};
  a.hidden = (const uint16_t*)hidden;
  a.num_tokens = T;
  a.hidden_size = H;
  a.intermediate_size = I;
  a.num_experts = E;
  a.top_k = K;
  a.topk_ids = ids;
  a.ids_dtype = MI355MOE_IDS_INT64;
  a.weight_layout = layout;
  a.topk_weights = wts;
  a.w1 = (const uint16_t*)w1;
  a.w2 = (const uint16_t*)w2;
  a.grad_out = (const uint16_t*)gout;
  a.grad_hidden = (uint16_t*)gh;
  a.grad_w1 = gw1;
  a.grad_w2 = gw2;
  a.grad_topk_weights = gp;
  a.weight_grad_dtype = grad_dtype;
  if (mx) {
    a.precision = MI355MOE_PRECISION_MXFP8;
    a.w1_scale = mk("w1_col_scale", (size_t)E * (H / 64) * 2 * I * 2);
    a.w2_scale = mk("w2_col_scale", (size_t)E * (I / 64) * H * 2);
    a.w1_row = mk("w1_row_data", (size_t)E * H * 2 * I);
    a.w2_row = mk("w2_row_data", (size_t)E * I * H);
    a.w1_row_scale = mk("w1_row_scale", (size_t)E * H * (2 * I / 32));
    a.w2_row_scale = mk("w2_row_scale", (size_t)E * I * (H / 32));
  }
  const size_t wsz = mi355moe_moe_backward_workspace_size(&a);
  uint8_t* ws = mk("workspace", wsz);
  g_expect = Expect();
  expect_rc(mi355moe_moe_backward(&a, ws, wsz, nullptr), 0, "moe_backward");
}

// The grouped-K GEMM on its own (as backward.hip calls it), operands [rows, M] / [rows, N] grouped by
// `counts`; MX operands with grouped packed column scales.
static void wgrad_direct(std::vector<int> counts, int M, int N, bool mx, int epi) {
  const int G = (int)counts.size();
  const auto glv = cumsum(counts);
  const int64_t R = glv.back();
  const int es = mx ? 1 : 2;
  uint8_t* A = mk("A", (size_t)R * M * es);
  uint8_t* B = mk("B", (size_t)R * N * es);
  const size_t groups = (size_t)(R + 63) / 64 + G;
  uint8_t* As = mx ? mk("A_col_scale", groups * M * 2) : nullptr;
  uint8_t* Bs = mx ? mk("B_col_scale", groups * N * 2) : nullptr;
  if (mx) {
    fill_e4m3(A, (size_t)R * M);
    fill_e4m3(B, (size_t)R * N);
    fill_codes(As, groups * M * 2);
    fill_codes(Bs, groups * N * 2);
  } else {
    fill_bf16(A, (size_t)R * M);
    fill_bf16(B, (size_t)R * N);
  }
  uint8_t* zero = mk("zero_row", (size_t)std::max(M, N) * es, 0);
  int64_t* gl = (int64_t*)mk("group_list", G * 8);
  memcpy(gl, glv.data(), G * 8);
  uint8_t* out = mk("dW", (size_t)G * M * N * (epi == EPI_STORE_F32 ? 4 : 2));
  GGParams p = {};
  p.A = A;
  p.lda_bytes = (int64_t)M * es;
  p.a_scale = As;
  p.B = B;
  p.b_row_bytes = (int64_t)N * es;
  p.b_scale = Bs;
  p.N = N;
  p.Ntot = N;
  p.m_rows = M;
  p.m_tiles = (M + GGBig::BM - 1) / GGBig::BM;
  p.n_tiles = (N + GGBig::BN - 1) / GGBig::BN;
  p.G = G;
  p.group_list = gl;
  p.C = out;
  p.ldc = N;
  p.c_group_stride = (int64_t)M * N;
  p.zero_row = zero;
  expect_rc(mi355_grouped_gemm_wgrad(p, epi, nullptr, mx), 0, "grouped_gemm_wgrad");
}

struct Scenario {
  const char* name;
  std::function<void()> run;
};

static std::vector<Scenario> scenarios() {
  const int L_EIO = MI355MOE_LAYOUT_EIO, L_EOI = MI355MOE_LAYOUT_EOI, L_GU = MI355MOE_LAYOUT_EIO_GU;
  const int BF = MI355MOE_PRECISION_BF16, MX = MI355MOE_PRECISION_MXFP8;
  std::vector<Scenario> s;
  // grouped GEMM C-ABI: ragged and empty groups, partial tiles, N not a multiple of the tile
  s.push_back({"gemm_bf16_eio", [=] { gemm_bf16({100, 0, 300, 1, 129}, 1024, 768, L_EIO); }});
  s.push_back({"gemm_bf16_eoi", [=] { gemm_bf16({100, 0, 300, 1, 129}, 1024, 768, L_EOI); }});
  s.push_back({"gemm_bf16_eio_narrow", [=] { gemm_bf16({3, 40, 0, 513}, 128, 200, L_EIO); }});
  s.push_back({"gemm_bf16_eoi_narrow", [=] { gemm_bf16({3, 40, 0, 513}, 128, 200, L_EOI); }});
  s.push_back({"gemm_mx_eio", [=] { gemm_mx({100, 0, 300, 1, 129}, 1024, 768, L_EIO); }});
  s.push_back({"gemm_mx_eoi", [=] { gemm_mx({100, 0, 300, 1, 129}, 1024, 768, L_EOI); }});
  s.push_back({"gemm_mx_eoi_long_k", [=] { gemm_mx({256, 256}, 2560, 272, L_EOI); }});
  s.push_back({"gemm_mx_eio_long_k", [=] { gemm_mx({256, 256}, 2560, 272, L_EIO); }});
  // decode-shaped groups (the 64-row tiles): at most 32 rows per group on average
  s.push_back({"gemm_bf16_eio_decode", [=] { gemm_bf16({5, 0, 17, 64, 1, 33, 0, 8}, 512, 1024, L_EIO); }});
  s.push_back({"gemm_bf16_eoi_decode", [=] { gemm_bf16({5, 0, 17, 64, 1, 33, 0, 8}, 512, 1024, L_EOI); }});
  s.push_back({"gemm_mx_eio_decode", [=] { gemm_mx({5, 0, 17, 64, 1, 33, 0, 8}, 1024, 512, L_EIO); }});
  s.push_back({"gemm_mx_eoi_decode", [=] { gemm_mx({5, 0, 17, 64, 1, 33, 0, 8}, 1024, 512, L_EOI); }});
  // the same decode shapes on the 256-row tiles (a build with the decode tiles off)
  auto decode_counts = [](int G, unsigned seed) {
    std::mt19937 r(seed);
    std::vector<int> c(G);
    for (auto& v : c) v = (int)(r() % 40);
    for (int i = 0; i < G / 3; ++i) c[r() % G] = 0;
    return c;
  };
  auto big = [](std::function<void()> f) {
    return [f] {
      g_force_big = true;
      f();
      g_force_big = false;
    };
  };
  s.push_back({"gemm_bf16_eio_decode_big", big([=] { gemm_bf16(decode_counts(64, 5), 1024, 768, L_EIO); })});
  s.push_back({"gemm_bf16_eoi_decode_big", big([=] { gemm_bf16(decode_counts(64, 5), 1024, 768, L_EOI); })});
  s.push_back({"gemm_mx_eio_decode_big", big([=] { gemm_mx(decode_counts(48, 6), 1024, 512, L_EIO); })});
  s.push_back({"moe_bf16_eio_decode_big", big([=] { moe_forward(32, 8, 64, 1024, 512, BF, L_EIO, 0.0); })});
  s.push_back({"moe_mx_eio_decode_big", big([=] { moe_forward(32, 8, 64, 1024, 512, MX, L_EIO, 0.0); })});
  s.push_back({"moe_bf16_gu_decode_big", big([=] { moe_forward(32, 8, 64, 1024, 512, BF, L_GU, 0.0); })});
  s.push_back({"moe_mx_gu_decode_big", big([=] { moe_forward(32, 8, 64, 1024, 512, MX, L_GU, 0.0); })});
  // decode tiles whose partial last round runs as column halves; the wrapper fails the scenario when
  // no item of it was a half
  auto halves = [](std::function<void()> f) {
    return [f] {
      const long before = g_half_items;
      f();
      if (g_half_items == before) CHECK_FAIL("no work item ran as a column half");
    };
  };
  s.push_back({"moe_mx_decode_halves", halves([=] { moe_forward(32, 8, 64, 1024, 512, MX, L_EIO, 0.0); })});
  s.push_back({"moe_mx_gu_decode_halves", halves([=] { moe_forward(32, 8, 64, 1024, 512, MX, L_GU, 0.0); })});
  s.push_back({"moe_bf16_decode_halves", halves([=] { moe_forward(32, 8, 64, 1024, 512, BF, L_EIO, 0.0); })});
  s.push_back({"moe_bf16_gu_decode_halves", halves([=] { moe_forward(32, 8, 64, 1024, 512, BF, L_GU, 0.0); })});
  s.push_back({"moe_mx_eoi_decode_halves", halves([=] { moe_forward(32, 8, 64, 1024, 512, MX, L_EOI, 0.0); })});
  // functional emulation (random operands; accumulators vs a reference GEMM). The EIO bf16 / MX and
  // EOI bf16 cases run on the GPU already and calibrate the instruction models.
  auto emu = [](std::function<void()> f) {
    return [f] {
      g_emulate = true;
      f();
      g_emulate = false;
    };
  };
  s.push_back({"emu_bf16_eio", emu([=] { gemm_bf16({70, 0, 129, 5}, 256, 512, L_EIO); })});
  s.push_back({"emu_bf16_eoi", emu([=] { gemm_bf16({70, 0, 129, 5}, 256, 512, L_EOI); })});
  s.push_back({"emu_mx_eio", emu([=] { gemm_mx({70, 0, 129, 5}, 1024, 256, L_EIO); })});
  s.push_back({"emu_mx_eoi", emu([=] { gemm_mx({70, 0, 129, 5}, 1024, 256, L_EOI); })});
  s.push_back({"emu_bf16_eio_decode", emu([=] { gemm_bf16({5, 0, 17, 64, 1, 33, 0, 8}, 256, 256, L_EIO); })});
  s.push_back({"emu_bf16_eoi_decode", emu([=] { gemm_bf16({5, 0, 17, 64, 1, 33, 0, 8}, 256, 256, L_EOI); })});
  s.push_back({"emu_mx_eio_decode", emu([=] { gemm_mx({5, 0, 17, 64, 1, 33, 0, 8}, 1024, 256, L_EIO); })});
  s.push_back({"emu_mx_eoi_decode", emu([=] { gemm_mx({5, 0, 17, 64, 1, 33, 0, 8}, 1024, 256, L_EOI); })});
  s.push_back({"emu_moe_mx_decode_halves", halves(emu([=] { moe_forward(16, 4, 16, 512, 256, MX, L_EIO, 0.0); }))});
  s.push_back({"emu_moe_bf16_decode_halves", halves(emu([=] { moe_forward(16, 4, 16, 512, 256, BF, L_EIO, 0.0); }))});
  s.push_back({"emu_moe_mx_gu_decode_halves", halves(emu([=] { moe_forward(16, 4, 16, 512, 256, MX, L_GU, 0.0); }))});
  s.push_back({"emu_wgrad_bf16", emu([=] { wgrad_direct({40, 0, 97, 33}, 256, 512, false, EPI_STORE_F32); })});
  s.push_back({"emu_wgrad_mx", emu([=] { wgrad_direct({40, 0, 97, 160}, 256, 256, true, EPI_STORE_F32); })});
  // the 8-wave configuration: through the library (grouped GEMM C-ABI, the MegaMoE forward in both
  // precisions and layouts, the no-allocation entry point) and directly on GGParams, with emulation
  s.push_back({"pp_gemm_bf16_eio", pp_route([=] { gemm_bf16({100, 0, 300, 1, 129, 600}, 1024, 768, L_EIO); })});
  s.push_back({"pp_gemm_bf16_eoi", pp_route([=] { gemm_bf16({100, 0, 300, 1, 129, 600}, 1024, 768, L_EOI); })});
  s.push_back({"pp_gemm_bf16_eio_narrow", pp_route([=] { gemm_bf16({3, 40, 0, 513}, 128, 200, L_EIO); })});
  s.push_back({"pp_gemm_bf16_many_items", pp_route([=] {
                 std::vector<int> c(40, 300);
                 gemm_bf16(c, 64, 2048, L_EOI);
               })});
  s.push_back({"pp_gemm_bf16_noalloc", pp_route([=] {
                 gemm_bf16({300, 0, 513, 77, 1}, 512, 512, L_EIO, true);
                 gemm_bf16({5, 400}, 256, 256, L_EOI, true);
               })});
  s.push_back({"pp_moe_bf16_eio_prefill", pp_route([=] { moe_forward(640, 2, 4, 256, 384, BF, L_EIO, 0.0); })});
  s.push_back({"pp_moe_bf16_eoi_prefill", pp_route([=] { moe_forward(640, 2, 4, 256, 384, BF, L_EOI, 0.0); })});
  s.push_back({"pp_moe_bf16_gu_prefill", pp_route([=] { moe_forward(640, 2, 4, 256, 384, BF, L_GU, 0.0); })});
  s.push_back({"pp_moe_mx_eio_prefill", pp_route([=] { moe_forward(640, 2, 4, 256, 384, MX, L_EIO, 0.0); })});
  s.push_back({"pp_moe_mx_gu_prefill", pp_route([=] { moe_forward(640, 2, 4, 256, 384, MX, L_GU, 0.0); })});
  s.push_back({"pp_moe_mx_gu_skewed", pp_route([=] { moe_forward(1500, 4, 12, 512, 256, MX, L_GU, 1.1); })});
  s.push_back({"pp_moe_bf16_gu_skewed", pp_route([=] { moe_forward(1500, 4, 12, 512, 256, BF, L_GU, 1.1); })});
  // variant "pp": the 8-wave kernel also on decode-shaped groups (1-40 rows, many empty)
  auto variant_pp = [](std::function<void()> f) {
    return [f] {
      g_variant = MI355_GG_VARIANT_PP;
      f();
      g_variant = 0;
    };
  };
  s.push_back({"pp_moe_mx_gu_decode_variant", pp_route(variant_pp([=] { moe_forward(32, 8, 64, 1024, 512, MX, L_GU, 0.0); }))});
  s.push_back({"pp_moe_bf16_eio_decode_variant", pp_route(variant_pp([=] { moe_forward(32, 8, 64, 1024, 512, BF, L_EIO, 0.0); }))});
  s.push_back({"pp_gemm_bf16_decode_variant", pp_route(variant_pp([=] { gemm_bf16(decode_counts(64, 5), 1024, 768, L_EOI); }))});
  s.push_back({"pp_bf16_kn_store", [=] { pp_gemm({70, 0, 129, 300, 1, 513}, 1024, 768, false, true, false, 0); }});
  s.push_back({"pp_mx_swiglu_gu", [=] { pp_gemm({70, 0, 129, 300, 1, 513}, 1024, 384, true, true, true, 1); }});
  s.push_back({"emu_pp_bf16_kn_store", emu([=] { pp_gemm({70, 0, 129, 300, 1}, 256, 512, false, true, false, 0); })});
  s.push_back({"emu_pp_bf16_nk_store", emu([=] { pp_gemm({70, 0, 129, 300, 1}, 256, 512, false, false, false, 0); })});
  s.push_back({"emu_pp_bf16_kn_store_256", emu([=] { pp_gemm({700, 33, 300}, 128, 256, false, true, false, 0); })});
  s.push_back({"emu_pp_bf16_kn_swiglu", emu([=] { pp_gemm({70, 0, 129, 300, 1}, 256, 256, false, true, true, 0); })});
  s.push_back({"emu_pp_bf16_kn_swiglu_gu", emu([=] { pp_gemm({70, 0, 129, 300, 1}, 256, 256, false, true, true, 1); })});
  s.push_back({"emu_pp_bf16_nk_swiglu", emu([=] { pp_gemm({70, 0, 129, 300, 1}, 256, 256, false, false, true, 0); })});
  s.push_back({"emu_pp_mx_store", emu([=] { pp_gemm({70, 0, 129, 300, 1}, 256, 512, true, true, false, 0); })});
  s.push_back({"emu_pp_mx_swiglu", emu([=] { pp_gemm({70, 0, 129, 300, 1}, 256, 256, true, true, true, 0); })});
  s.push_back({"emu_pp_mx_swiglu_gu", emu([=] { pp_gemm({70, 0, 257, 1, 511}, 256, 256, true, true, true, 1); })});
  // the skinny 384 x 128 MX tile (switched on for the scenario): the groups of 257..384 rows on it,
  // the others on the 256 x 256 tile, in two launches
  auto skinny = [](std::function<void()> f) {
    return [f] {
      const long before = g_pp_skinny_launches;
      setenv("MI355MOE_PP_SKINNY", "1", 1);
      f();
      unsetenv("MI355MOE_PP_SKINNY");
      if (g_pp_skinny_launches == before) CHECK_FAIL("no launch ran on the 384 x 128 tile");
    };
  };
  s.push_back({"emu_pp_mx_skinny_store",
               emu(skinny([=] { pp_gemm({300, 70, 384, 257, 385, 0, 256}, 256, 512, true, true, false, 0); }))});
  s.push_back({"emu_pp_mx_skinny_swiglu",
               emu(skinny([=] { pp_gemm({300, 70, 384, 257, 385, 0, 256}, 256, 256, true, true, true, 0); }))});
  s.push_back({"emu_pp_mx_skinny_swiglu_gu",
               emu(skinny([=] { pp_gemm({300, 70, 384, 257, 385, 0, 256}, 256, 256, true, true, true, 1); }))});
  // bf16 with K-contiguous weights: beside the 320-row tiles (groups averaging at most 320 rows) and
  // beside the 256-row ones
  s.push_back({"emu_pp_bf16_nk_skinny_store_320",
               emu(skinny([=] { pp_gemm({330, 70, 384, 321, 385, 0, 200, 300}, 256, 512, false, false, false, 0); }))});
  s.push_back({"emu_pp_bf16_nk_skinny_swiglu_320",
               emu(skinny([=] { pp_gemm({330, 70, 384, 321, 385, 0, 200, 300}, 256, 256, false, false, true, 0); }))});
  s.push_back({"emu_pp_bf16_nk_skinny_store_256",
               emu(skinny([=] { pp_gemm({300, 500, 384, 257, 600, 350}, 256, 512, false, false, false, 0); }))});
  s.push_back({"emu_pp_bf16_nk_skinny_swiglu_256",
               emu(skinny([=] { pp_gemm({300, 500, 384, 257, 600, 350}, 256, 256, false, false, true, 0); }))});
  s.push_back({"emu_pp_bf16_kn_skinny_store_320",
               emu(skinny([=] { pp_gemm({330, 70, 384, 321, 385, 0, 200, 300}, 256, 512, false, true, false, 0); }))});
  s.push_back({"emu_pp_bf16_kn_skinny_swiglu_256",
               emu(skinny([=] { pp_gemm({300, 500, 384, 257, 600, 350}, 256, 256, false, true, true, 0); }))});
  s.push_back({"emu_pp_bf16_kn_skinny_swiglu_gu_320",
               emu(skinny([=] { pp_gemm({330, 70, 384, 321, 385, 0, 200, 300}, 256, 256, false, true, true, 1); }))});
  s.push_back({"pp_moe_bf16_gu_skinny", pp_route(skinny([=] { moe_forward(704, 2, 4, 256, 384, BF, L_GU, 0.0); }))});
  s.push_back({"pp_moe_bf16_eio_skinny", pp_route(skinny([=] { moe_forward(640, 2, 4, 256, 384, BF, L_EIO, 0.0); }))});
  s.push_back({"pp_moe_bf16_eoi_skinny", pp_route(skinny([=] { moe_forward(704, 2, 4, 256, 384, BF, L_EOI, 0.0); }))});
  s.push_back({"pp_moe_mx_eio_skinny", pp_route(skinny([=] { moe_forward(640, 2, 4, 256, 384, MX, L_EIO, 0.0); }))});
  s.push_back({"pp_moe_mx_gu_skinny", pp_route(skinny([=] { moe_forward(640, 2, 4, 256, 384, MX, L_GU, 0.0); }))});
  // the switched-off paths stay off without their environment variables
  s.push_back({"gate_skinny_off", pp_route([=] {
                 const long before = g_pp_skinny_launches;
                 moe_forward(640, 2, 4, 256, 384, MX, L_GU, 0.0);
                 if (g_pp_skinny_launches != before) CHECK_FAIL("the 384 x 128 tile ran while switched off");
               })});
  s.push_back({"gate_decode_prep_off", [=] {
                 const long before = g_preps;
                 unsetenv("MI355MOE_DECODE_PREP");
                 moe_forward(32, 8, 64, 1024, 512, MX, L_GU, 0.0);
                 setenv("MI355MOE_DECODE_PREP", "1", 1);
                 if (g_preps != before) CHECK_FAIL("the one-launch decode prologue ran while switched off");
               }});
  s.push_back({"pp_moe_mx_gu_skinny_none",  // no group in the range: the 384 x 128 launch has no work
               pp_route(skinny([=] { moe_forward(700, 4, 16, 256, 256, MX, L_GU, 0.0); }))});
  s.push_back({"pp_moe_mx_gu_skinny_skewed",
               pp_route(skinny([=] { moe_forward(1500, 4, 12, 512, 256, MX, L_GU, 1.1); }))});
  s.push_back({"emu_moe_bf16_numerics_clamp", emu([=] { moe_forward(16, 4, 16, 512, 256, BF, L_EIO, 0.0, 0, 7.0f); })});
  s.push_back({"emu_moe_bf16_numerics_after_silu",
               emu([=] { moe_forward(16, 4, 16, 512, 256, BF, L_EOI, 0.0, MI355MOE_NUMERICS_CLAMP_AFTER_SILU, 7.0f); })});
  s.push_back({"emu_moe_bf16_probs_before_fc2",
               emu([=] { moe_forward(16, 4, 16, 512, 256, BF, L_EIO, 0.0, MI355MOE_NUMERICS_PROBS_BEFORE_FC2); })});
  s.push_back({"mut_epi_exp", epi_mutant(1, halves(emu([=] { moe_forward(16, 4, 16, 512, 256, BF, L_EIO, 0.0); })))});
  s.push_back({"mut_epi_rounding", epi_mutant(2, halves(emu([=] { moe_forward(16, 4, 16, 512, 256, MX, L_EIO, 0.0); })))});
  s.push_back({"mut_epi_scale", epi_mutant(3, halves(emu([=] { moe_forward(16, 4, 16, 512, 256, MX, L_EIO, 0.0); })))});
  s.push_back({"mut_pp_copy_offset", pp_mutant(1, emu([=] { pp_gemm({70, 129}, 256, 256, false, true, false, 0); }))});
  s.push_back({"mut_pp_copy_oob", pp_mutant(2, [=] { pp_gemm({70, 129}, 256, 256, false, true, false, 0); })});
  s.push_back({"mut_pp_copy_skipped", pp_mutant(3, [=] { pp_gemm({70, 129}, 256, 256, true, true, false, 0); })});
  s.push_back({"mut_pp_staging", pp_mutant(4, emu([=] { pp_gemm({70, 129}, 256, 256, false, true, true, 0); }))});
  s.push_back({"mut_pp_shuffle", pp_mutant(5, emu([=] { pp_gemm({70, 129}, 256, 256, true, true, true, 1); }))});
  s.push_back({"mut_pp_rounding", pp_mutant(6, emu([=] { pp_gemm({70, 129}, 256, 256, true, true, true, 1); }))});
  // many groups: the tile prefix comes from global memory past the LDS copy
  s.push_back({"gemm_bf16_many_groups", [=] {
                 std::vector<int> c(1100, 0);
                 for (size_t i = 0; i < c.size(); i += 3) c[i] = 1 + (int)(i % 7);
                 gemm_bf16(c, 64, 256, L_EIO);
               }});
  // the no-allocation entry point: the tile plan in the static array, looked up once; a second,
  // smaller call reads only what it planned
  s.push_back({"gemm_bf16_noalloc", [=] {
                 gemm_bf16({300, 0, 513, 77, 1}, 512, 512, L_EIO, true);
                 gemm_bf16({5, 40}, 256, 256, L_EOI, true);
                 if (g_symbol_lookups != 1) CHECK_FAIL("scratch address looked up %ld times", g_symbol_lookups);
               }});
  // MegaMoE forward, bf16 and MX, both layouts; prefill-like and decode-like routing
  s.push_back({"moe_bf16_eio", [=] { moe_forward(96, 4, 16, 512, 256, BF, L_EIO, 1.1); }});
  s.push_back({"moe_bf16_eoi", [=] { moe_forward(96, 4, 16, 512, 256, BF, L_EOI, 1.1); }});
  s.push_back({"moe_bf16_eio_prefill", [=] { moe_forward(640, 2, 4, 256, 384, BF, L_EIO, 0.0); }});
  s.push_back({"moe_mx_eio", [=] { moe_forward(96, 4, 16, 512, 256, MX, L_EIO, 1.1); }});
  s.push_back({"moe_mx_eoi", [=] { moe_forward(96, 4, 16, 512, 256, MX, L_EOI, 1.1); }});
  s.push_back({"moe_mx_eoi_prefill", [=] { moe_forward(640, 2, 4, 256, 384, MX, L_EOI, 0.0); }});
  s.push_back({"moe_mx_eio_prefill", [=] { moe_forward(640, 2, 4, 256, 384, MX, L_EIO, 0.0); }});
  s.push_back({"moe_mx_gu_prefill", [=] { moe_forward(640, 2, 4, 256, 384, MX, L_GU, 0.0); }});
  s.push_back({"moe_bf16_gu", [=] { moe_forward(96, 4, 16, 512, 256, BF, L_GU, 1.1); }});
  s.push_back({"moe_bf16_numerics_clamp", [=] { moe_forward(96, 4, 16, 512, 256, BF, L_EIO, 1.1, 0, 7.0f); }});
  s.push_back({"moe_bf16_numerics_after_silu",
               [=] { moe_forward(96, 4, 16, 512, 256, BF, L_EOI, 1.1, MI355MOE_NUMERICS_CLAMP_AFTER_SILU, 7.0f); }});
  s.push_back({"moe_bf16_probs_before_fc2",
               [=] { moe_forward(640, 2, 4, 256, 384, BF, L_EIO, 0.0, MI355MOE_NUMERICS_PROBS_BEFORE_FC2); }});
  // expert backward
  s.push_back({"bwd_eio_f32", [=] { moe_backward(96, 4, 8, 256, 128, L_EIO, MI355MOE_GRAD_FP32, 1.1); }});
  s.push_back({"bwd_eoi_bf16", [=] { moe_backward(96, 4, 8, 256, 128, L_EOI, MI355MOE_GRAD_BF16, 1.1); }});
  s.push_back({"bwd_eio_bf16_prefill", [=] { moe_backward(300, 2, 3, 384, 256, L_EIO, MI355MOE_GRAD_BF16, 0.0); }});
  s.push_back({"bwd_mx_f32", [=] { moe_backward(96, 4, 8, 512, 256, L_EIO, MI355MOE_GRAD_FP32, 1.1, true); }});
  s.push_back({"bwd_mx_bf16_prefill", [=] { moe_backward(300, 2, 3, 1024, 512, L_EIO, MI355MOE_GRAD_BF16, 0.0, true); }});
  return s;
}

int main(int argc, char** argv) {
  // every optional path on: also the one-launch decode prologue (read once by the library)
  setenv("MI355MOE_DECODE_PREP", "1", 1);
  const auto all = scenarios();
  if (argc == 2 && std::string(argv[1]) == "--list") {
    for (const auto& sc : all) printf("%s\n", sc.name);
    return 0;
  }
  int ran = 0;
  for (const auto& sc : all) {
    bool pick = argc < 2;
    for (int i = 1; i < argc; ++i) pick |= std::string(argv[i]) == sc.name;
    if (!pick) continue;
    g_scenario = sc.name;
    const long e0 = g_errors, c0 = g_copies, i0 = g_items, m0 = g_gemms, u0 = g_emulated_items, p0 = g_preps,
               q0 = g_epilogue_items;
    sc.run();
    free_all();
    printf("%-32s %s  gemms=%ld items=%ld copies=%ld emulated=%ld epilogues=%ld preps=%ld\n", sc.name,
           g_errors == e0 ? "ok" : "FAILED", g_gemms - m0, g_items - i0, g_copies - c0, g_emulated_items - u0,
           g_epilogue_items - q0, g_preps - p0);
    fflush(stdout);
    ++ran;
  }
  if (ran == 0) {
    fprintf(stderr, "no scenario matched\n");
    return 2;
  }
  printf("%d scenarios, %ld errors\n", ran, g_errors);
  return g_errors ? 1 : 0;
}
