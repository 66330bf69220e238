// 8-wave ping-pong grouped GEMM (gemm_pp.hip): tile configurations, work-item decode, the per-lane
// copy plan and copy issue, the LDS fragment reads, the MFMAs and the epilogues.
//
// Everything here is __host__ __device__ and reaches the hardware only through a policy type `O`:
// PpDev (below) issues the gfx950 instructions (direct-to-LDS loads, readfirstlane, LDS loads and
// stores, the transposing LDS loads, the MFMAs, lane shuffles); the host-side checker under
// tests/native instantiates the same code with a policy that records and bounds-checks every copy,
// lands it in an emulated LDS, emulates the lane-crossing instructions and the MFMAs and checks
// every global store, so the kernel's addressing and data path are replayed on the CPU before they
// run on a GPU. Policy methods that only the device needs (`opaque`, `uni`) are identities on the
// host.
//
// Work list: every (group, BM-row m-tile, BN-column n-tile) is one work item of the groups the launch
// takes (all, or either side of the skinny tile's row range); the m-tiles of a group come from
// group_list at the kernel's own tile height (tile prefix and group row ends in LDS). Workgroup b starts at item (b % 8) * (grid / 8) + b / 8 and steps by the grid, so each XCD
// runs a contiguous run of items (m fastest) and the n-tiles that re-read one expert's activation
// rows run at the same time on one XCD and share its L2.
//
// Workgroup: 512 threads = 8 wavefronts, two per SIMD. Tiles are BM x 256 (BM = 320 for bf16, 256
// for MXFP8), or 384 x 128 (the MXFP8 skinny tile). The waves form two groups, 0-3 and 4-7, one wave
// of each on every SIMD; on the 256-column tiles wave w computes columns 64 * (w % 4) ..+63 of the
// 32-row blocks 2 mi + w / 4 (mi < BM / 64), on the 128-column tile columns 64 * (w % 2) ..+63 of the
// blocks 4 mi + w / 4 + 2 ((w % 4) / 2) (mi < 3): 2 x MI blocks of 32 x 32 (bf16
// v_mfma_f32_32x32x16_bf16, MXFP8 v_mfma_scale_f32_32x32x64_f8f6f4). The row blocks alternate between
// the groups and the activation copies between the waves, so a tile that is not full keeps the two
// groups and the eight waves evenly loaded; bf16 waves skip the MFMAs of row blocks past the item's
// rows.
//
// K stages are 128 bytes per row (64 bf16 or 128 e4m3): whole 128-byte lines per row and stage. A
// stage is 64 KB of operands, so the LDS ring has two slots: the copies of stage q + 1 go out at the
// start of the interval in which stage q is used, into the slot that stage q - 1 left.
//
// LDS layouts (16-byte chunks, XOR swizzled against bank conflicts):
//   K-contiguous rows (activations; EOI weights): row r at r * 128, chunk c at c ^ ((r >> 1) & 7),
//     read with ds_read_b128;
//   N-contiguous weights (EIO bf16, MX col_data): K row k of the stage holds the tile's columns; bf16
//     chunk c at c ^ ((k & 7) << 1) (512-byte rows; 256 on the 128-column tile), e4m3 chunk c at
//     c ^ (k & 15) (256-byte rows; the 128-column tile: c ^ (k & 7), 128-byte rows), read with
//     ds_read_b64_tr_b16 / ds_read_b64_tr_b8;
//   MX scales of a stage: code j (0..3) of tile row r at j * 512 + row0 % 4 + r (from the
//     stage-major code planes of the activation scales: two 256-byte runs per code from the 4-aligned
//     address at or below the tile's first row); weight tile column j's two codes of 64-K step s at
//     s * 2 BN + j * 2 (the MX root's col_scale pairs).
//
// Epilogues: bf16 store, SwiGLU -> bf16 (each 32 x 32 block through a wave-private LDS staging block,
// so the global stores are 16 bytes per lane), for MX inputs SwiGLU -> fp32 (staged 16 rows at a
// time, 32-byte stores) and SwiGLU -> MXFP8 (the same staging; the 4 lanes of a row reduce its
// 32-column block maximum and write 8 e4m3 bytes each, the block's scale code goes to the
// stage-major code planes GMM2 reads). For SwiGLU the 64 weight columns of a wave are 32 gate then the matching
// 32 up columns, so a lane holds gate and up of the same output element.
#pragma once
#include "common.h"
#include "gemm.h"

namespace pp {

constexpr int KB = 128;  // bytes of K per row and stage
constexpr int S = 2;     // ring slots
constexpr int WAVES = 8, THREADS = 64 * WAVES;
constexpr int WN = 64, NI = WN / 32;
// MX activation scales of a stage: 4 code planes of 512 bytes (the tile rows from the 4-aligned row
// at or below the first one; 512 covers tiles of up to 509 rows)
constexpr int AS_PLANE = 512;
constexpr int AS_BYTES = 4 * AS_PLANE;

// The skinny tile (384 x 128) takes the groups of more rows than the other launch's tile height and
// at most SKINNY_HI. Groups a launch takes: SEL_ALL; SEL_NOT_SKINNY (all but those, on a tile of BM
// rows); SEL_SKINNY_256 / SEL_SKINNY_320 (only those, beside a launch on 256- / 320-row tiles).
constexpr int SKINNY_HI = 384;
enum { SEL_ALL = 0, SEL_NOT_SKINNY = 1, SEL_SKINNY_256 = 2, SEL_SKINNY_320 = 3 };
template <int SEL>
constexpr bool sel_skinny = SEL >= SEL_SKINNY_256;
template <int SEL, int BM>
MI355_HD bool sel_takes(int64_t rows) {
  if constexpr (SEL == SEL_ALL) return true;
  constexpr int lo = SEL == SEL_SKINNY_256 ? 256 : SEL == SEL_SKINNY_320 ? 320 : BM;
  const bool skinny = rows > lo && rows <= SKINNY_HI;
  return sel_skinny<SEL> ? skinny : !skinny;
}

// Tile shape and LDS layout. Tiles are 256 x 256; 320 x 256 for bf16 GEMMs whose groups average at
// most 320 rows (TALL): each m-tile streams its group's weights, whose lines miss L2, and the
// workgroup's memory requests in flight are what bounds the kernel, so an expert of 257..320 routed
// rows (DeepSeek-V3 prefill routes 256 on average, with a wide spread) is one m-tile instead of a
// full one and a short one that streams the weights again. When groups are large multiples of 256
// rows the fifth row block costs more than the tiles it saves. MX tiles of 256 rows have no registers
// left for a fifth row block. SK: the skinny 384 x 128 tile (each wave 3 row blocks x 64 columns, two
// waves of a group per column range), which streams the weights of an expert of up to 384 rows once.
template <bool MX_, bool TALL, bool SK = false>
struct Cfg {
  static constexpr bool MX = MX_;
  static constexpr bool SKINNY = SK;
  static constexpr int BM = SKINNY ? 384 : (MX || !TALL) ? 256 : 320;
  static constexpr int BN = SKINNY ? 128 : 256;
  static constexpr int WQN = BN / WN;            // waves of a group across the tile's columns
  static constexpr int RBS = 2 * (4 / WQN);      // row-block stride of a wave
  static constexpr int MI = BM / (32 * RBS);     // 32-row blocks per wave
  static constexpr int A_BYTES = BM * KB, B_BYTES = BN * KB, BS_BYTES = 2 * BN * 2;
  static constexpr int CPW_A = A_BYTES / 1024 / WAVES;  // 1 KB activation copies per wave and stage
  static constexpr int CPW_B = B_BYTES / 1024 / WAVES;  // 1 KB weight copies per wave and stage
  static constexpr int B_CH_LOG = SKINNY ? 3 : 4;       // MX weight K rows: BN bytes = 1 << B_CH_LOG chunks
  // wave w: columns 64 wq_of(w) ..+63, row blocks RBS mi + rbo_of(w); the groups are w / 4
  MI355_HD static int wq_of(int w) { return w & (WQN - 1); }
  MI355_HD static int rbo_of(int w) { return (w >> 2) + 2 * ((w & 3) / WQN); }
  static constexpr int B_OFF = A_BYTES, AS_OFF = B_OFF + B_BYTES, BS_OFF = AS_OFF + AS_BYTES;
  static constexpr int SLOT = MX ? BS_OFF + BS_BYTES : AS_OFF;
  static constexpr int PREFIX_OFF = S * SLOT;
  static constexpr int PREFIX_MAX = BM > 256 ? 512 : 1024;  // groups whose tile prefix and row ends are in LDS
  static constexpr int ROWS_OFF = PREFIX_OFF + (PREFIX_MAX + 1) * 4;
  // a wave's epilogue staging: 16 rows of a 32-column bf16 block (MX: 16 rows of 32 fp32 columns)
  static constexpr int EPI_BLOCK = MX ? 2048 : 1024;
  static constexpr int EPI_OFF = (ROWS_OFF + PREFIX_MAX * 4 + 15) & ~15;
  static constexpr int TOTAL = EPI_OFF + WAVES * EPI_BLOCK;
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
  static_assert(SLOT % 16 == 0, "copy destinations are 16-byte aligned");
  static_assert(A_BYTES % (1024 * WAVES) == 0, "whole 1 KB activation copies per wave");
  static_assert(B_BYTES % (1024 * WAVES) == 0 && (BN >> B_CH_LOG) == 16, "whole 1 KB weight copies per wave");
  static_assert(BM + 3 <= AS_PLANE, "a code plane run covers the tile");
  static_assert(MI * 32 * RBS == BM && RBS * WQN == 8, "wave geometry");
};

// The device policy: the gfx950 instructions behind the shared code.
struct PpDev {
  MI355_DEV static uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
  MI355_DEV static int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
  // A pointer known to be wave-uniform, held in scalar registers.
  MI355_DEV static const uint8_t* uni_ptr(const uint8_t* ptr) {
    const uint64_t v = (uint64_t)(uintptr_t)ptr;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  }
  // The value through an empty asm: offsets derived from it are recomputed where they are used
  // instead of being hoisted into registers held across a loop.
  MI355_DEV static int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
  }
  // Direct global -> LDS copies: lane i writes its 16 (4) bytes at LDS address M0 + 16 i (4 i).
  // Inline assembly, so that the compiler does not treat the copy as an alias of every later LDS read
  // (its builtin makes it wait for all outstanding loads before the next ds_read). The source is a
  // wave-uniform base in scalar registers plus a 32-bit per-lane offset; m0 is an LDS address (and
  // declared clobbered, so the compiler keeps no value of its own in it across a copy).
  MI355_DEV static void dma16(const uint8_t* base, uint32_t off, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0)
                 : "memory", "m0");
  }
  MI355_DEV static void dma4(const uint8_t* base, uint32_t off, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(m0)
                 : "memory", "m0");
  }
  template <class T>
  MI355_DEV static T lds(const uint8_t* p) {
    return *(const __attribute__((address_space(3))) T*)p;
  }
  // the epilogue's staging block: an LDS pointer, and loads / stores through it
  using lds_ptr = __attribute__((address_space(3))) uint8_t*;
  MI355_DEV static lds_ptr lds_base(uint8_t* p) { return (lds_ptr)p; }
  template <class T>
  MI355_DEV static void lds_store(lds_ptr p, T v) {
    *(__attribute__((address_space(3))) T*)p = v;
  }
  template <class T>
  MI355_DEV static T lds_load(lds_ptr p) {
    return *(__attribute__((address_space(3))) T*)p;
  }
  template <class T>
  MI355_DEV static void store(void* p, T v) {
    *(T*)p = v;
  }
  MI355_DEV static v4s tr16(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
  }
  MI355_DEV static v2i tr8(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)p);
  }
  MI355_DEV static void mfma_bf16(v8bf a, v8bf b, v16f& acc) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
  }
  MI355_DEV static void mfma_f8(v8i a, v8i b, v16f& acc, int sa, int sb) {
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc, 0, 0, 0, sa, 0, sb);
  }
  MI355_DEV static float expf(float x) { return __expf(x); }
  MI355_DEV static float shfl_xor(float v, int m) { return __shfl_xor(v, m); }
  MI355_DEV static uint32_t e4m3(float v) { return f32_to_e4m3_inrange(v); }
};

// Tile column j (0..BN-1) -> weight column; SwiGLU: wave tile q's 64 columns are gate columns
// nt * BN / 2 + 32 q .. +31, then the up columns I + the same.
// With the gate/up interleaved weight layout the projection column goes through gate_up_col.
template <int BN>
MI355_HD int tile_col(int j, int nt, int I, bool swiglu, int gu) {
  if (!swiglu) return nt * BN + j;
  const int q = j >> 6, jj = j & 63;
  const int base = nt * (BN / 2) + q * 32;
  return gate_up_col(jj < 32 ? base + jj : I + base + (jj - 32), I, gu);
}

struct Item {
  int64_t row0;  // first routed row of the tile
  int rows;      // valid rows (1..BM)
  int nt;        // n-tile
  int g;         // group
};

// Work item L from the tile prefix and the groups' row ends, both in LDS (LDS reads only: a global
// or generic load here would make the wave wait for all of its outstanding copies).
template <class C, class O>
MI355_HD void decode(const GGParams& p, const uint8_t* smem, int L, Item& it) {
  constexpr int BM = C::BM;
  auto prefix = [&](int g) { return O::template lds<int32_t>(smem + C::PREFIX_OFF + 4 * g); };
  auto rows = [&](int g) { return O::template lds<int32_t>(smem + C::ROWS_OFF + 4 * g); };
  int lo = 0, hi = p.G - 1;
  while (lo < hi) {  // largest g with prefix[g] * n_tiles <= L
    const int mid = (lo + hi + 1) >> 1;
    if (prefix(mid) * p.n_tiles <= L) lo = mid; else hi = mid - 1;
  }
  const int g = O::uni(lo);
  const int mtiles = O::uni(prefix(g + 1) - prefix(g));
  const int local = L - O::uni(prefix(g)) * p.n_tiles;
  const int nt = local / mtiles;
  const int mt = local - nt * mtiles;
  const int64_t row_begin = g == 0 ? 0 : O::uni(rows(g - 1));
  const int64_t row_end = O::uni(rows(g));
  it.g = g;
  it.nt = nt;
  it.row0 = row_begin + (int64_t)mt * BM;
  const int64_t left = row_end - it.row0;
  it.rows = O::uni((int)(left < BM ? left : BM));
}

// Copy sources of one work item: wave-uniform bases of stage 0 (stage k adds k * the stride) and
// per-lane 32-bit offsets (the activations, one group's weights and the scale arrays are below
// 4 GiB, which mi355_gg_pp_applies checks).
// Only the gathered activation offsets are kept per lane; the weight and scale offsets are functions
// of the lane and the item's n-tile, recomputed for every stage (holding them across the K loop
// pushed the MX kernels past their registers, and a spill reload between the copies waits for all
// of them).
template <int CPW_A>
struct Plan {
  const uint8_t* a_base;
  const uint8_t* b_base;
  const uint8_t* s_base;   // MX: activation code plane run (every wave)
  const uint8_t* bs_base;  // MX: the group's weight scales (waves 0-3; waves 4-7 repeat them)
  uint32_t ao[CPW_A];
  int a_copies;  // activation copies of this wave (8-row groups past the item's rows are skipped)
  int nt;        // the item's n-tile
  int64_t b_stride, s_stride, b_scale_stride;
};

// Activation and EOI-weight copies: copy i of a stage covers rows 8 i ..+7, lane l row
// 8 i + l / 8 and LDS position l % 8, which holds chunk (l % 8) ^ ((row >> 1) & 7).
MI355_HD int row_of(int i, int lane) { return i * 8 + (lane >> 3); }
MI355_HD int chunk_of(int r, int lane) { return (lane & 7) ^ ((r >> 1) & 7); }

template <class C, bool B_KN, bool SWIGLU, class O>
MI355_HD void make_plan(const GGParams& p, const Item& it, int wave, int lane, Plan<C::CPW_A>& pl) {
  constexpr bool MX = C::MX;
  constexpr int ESIZE = MX ? 1 : 2, CPW = C::CPW_A;
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int r = row_of(j * WAVES + wave, lane);
    const int rr = r < it.rows ? r : it.rows - 1;
    const int64_t routed = it.row0 + rr;
    const int64_t src = p.a_row_index ? (int64_t)(p.a_row_index[routed] / p.a_row_div) : routed;
    pl.ao[j] = (uint32_t)(src * p.lda_bytes + chunk_of(r, lane) * 16);
  }
  pl.a_base = O::uni_ptr(p.A);
  {
    // copies of 8-row groups holding rows of the item: the wave's are j * WAVES + wave
    const int groups = (it.rows + 7) / 8;
    const int n = (groups - wave + WAVES - 1) / WAVES;
    pl.a_copies = O::uni(n < 0 ? 0 : (n > CPW ? CPW : n));
  }
  pl.b_base = O::uni_ptr(p.B + (int64_t)it.g * p.b_group_stride);
  pl.nt = O::uni(it.nt);
  pl.b_stride = B_KN ? (int64_t)(KB / ESIZE) * p.b_row_bytes : KB;
  pl.s_base = pl.a_base;
  pl.bs_base = pl.a_base;
  pl.s_stride = 0;
  if constexpr (MX) {
    // code plane wave / 2, bytes 256 (wave % 2) + 4 lane from the 4-aligned row at or below row0
    // (rows past the item read the next rows or the planes' padding)
    pl.s_base = O::uni_ptr(p.a_scale + (wave >> 1) * (p.a_scale_stage_stride >> 2) + (it.row0 & ~(int64_t)3));
    pl.s_stride = p.a_scale_stage_stride;
    pl.bs_base = O::uni_ptr(p.b_scale + (int64_t)it.g * p.b_scale_group_stride);
    pl.b_scale_stride = (int64_t)p.Ntot * 4;  // two 64-K steps per stage
  }
}

template <class C, bool B_KN, bool SWIGLU>
MI355_HD uint32_t b_off(const GGParams& p, int nt, int i, int lane) {
  if constexpr (!B_KN) {  // K-contiguous weights: like the activations, one weight row per tile column
    const int r = row_of(i, lane);
    int wc = tile_col<C::BN>(r, nt, p.N, SWIGLU, p.gate_up_interleaved);
    if (wc >= p.Ntot) wc = p.Ntot - 1;
    return (uint32_t)wc * (uint32_t)p.b_row_bytes + (uint32_t)(chunk_of(r, lane) * 16);
  } else if constexpr (C::MX) {
    // K rows of BN bytes (16 or 8 chunks): copy i covers K rows (4 or 8) i ..
    constexpr int LG = C::B_CH_LOG, M = (1 << LG) - 1;
    const int L16 = i * 64 + lane;
    const int k = L16 >> LG;
    const int c = (L16 & M) ^ (k & M);
    int wc = tile_col<C::BN>(c * 16, nt, p.N, SWIGLU, p.gate_up_interleaved);
    if (wc > p.Ntot - 16) wc = p.Ntot - 16;
    return (uint32_t)k * (uint32_t)p.b_row_bytes + (uint32_t)wc;
  } else {
    // K rows of 2 BN bytes (512: copy i covers K rows 2 i, 2 i + 1; 256 on the 128-column tile)
    constexpr int LG = C::SKINNY ? 4 : 5, M = (1 << LG) - 1;
    const int L16 = i * 64 + lane;
    const int k = L16 >> LG;
    const int c = (L16 & M) ^ ((k & 7) << 1);
    int wc = tile_col<C::BN>(c * 8, nt, p.N, SWIGLU, p.gate_up_interleaved);
    if (wc > p.Ntot - 8) wc = p.Ntot - 8;
    return (uint32_t)k * (uint32_t)p.b_row_bytes + (uint32_t)wc * 2u;
  }
}

// The copies of stage k into the ring slot at LDS address `slot`. `lane` is made opaque per stage,
// so that the offsets derived from it are recomputed here rather than hoisted out of the K loop into
// registers.
template <class C, bool B_KN, bool SWIGLU, class O>
MI355_HD void issue_stage(const GGParams& p, const Plan<C::CPW_A>& pl, int k, uint32_t slot, int wave, int lane_in) {
  constexpr bool MX = C::MX;
  constexpr int CPW = C::CPW_A;
  const int lane = O::opaque(lane_in);
  const uint8_t* ab = O::uni_ptr(pl.a_base + (int64_t)k * KB);
  const uint8_t* bb = O::uni_ptr(pl.b_base + (int64_t)k * pl.b_stride);
  // (the waits are for all outstanding copies, so a wave may issue fewer; LDS rows that are not
  // refilled hold stale data that only feeds accumulator rows the epilogue does not store)
#pragma unroll
  for (int j = 0; j < CPW; ++j)
    if (j < pl.a_copies) O::dma16(ab, pl.ao[j], O::uni(slot + (j * WAVES + wave) * 1024));
#pragma unroll
  for (int j = 0; j < C::CPW_B; ++j)
    O::dma16(bb, b_off<C, B_KN, SWIGLU>(p, pl.nt, wave * C::CPW_B + j, lane),
             O::uni(slot + C::B_OFF + (wave * C::CPW_B + j) * 1024));
  if constexpr (MX) {
    // activation code planes: plane wave / 2, bytes 256 (wave % 2) + 4 lane of the item's run;
    // col_scale [G, K/64, Ntot, 2]: wave w (and w + 4) copies 64-K step (w >> 1) & 1, tile columns
    // 128 (w & 1) ..+127 (a 128-column tile: the waves with w & 1 == 0 only), to step * 2 BN
    const uint32_t so = (uint32_t)((wave & 1) * 256 + lane * 4);
    int wc = tile_col<C::BN>((wave & 1) * 128 + lane * 2, pl.nt, p.N, SWIGLU, p.gate_up_interleaved);
    if (wc > p.Ntot - 2) wc = p.Ntot - 2;
    const uint32_t bso = (uint32_t)((((wave >> 1) & 1) * p.Ntot + wc) * 2);
    O::dma4(O::uni_ptr(pl.s_base + (int64_t)k * pl.s_stride), so,
            O::uni(slot + C::AS_OFF + (wave >> 1) * AS_PLANE + (wave & 1) * 256));
    if (C::BN == 256 || (wave & 1) == 0)
      O::dma4(O::uni_ptr(pl.bs_base + (int64_t)k * pl.b_scale_stride), bso,
              O::uni(slot + C::BS_OFF + ((wave >> 1) & 1) * (2 * C::BN) + (wave & 1) * 256));
  }
}

// LDS offset of 16-byte chunk c of K-contiguous row r
MI355_HD int chunk_off(int r, int c) { return r * KB + ((c ^ ((r >> 1) & 7)) << 4); }

// Operand fragments of one half-step (64 bytes of K).
template <bool MX, bool B_KN, int MI> struct Frags;
template <int MI> struct Frags<false, false, MI> { v8bf a[2][MI], b[2][NI]; };
template <int MI> struct Frags<false, true, MI> { v8bf a[2][MI]; v4s bl[2][NI], bh[2][NI]; };
template <int MI> struct Frags<true, false, MI> { v4i al[MI], ah[MI], bl[NI], bh[NI]; int sa[MI], sb[NI]; };
template <int MI> struct Frags<true, true, MI> { v4i al[MI], ah[MI]; v2i bp[NI][4]; int sa[MI], sb[NI]; };

// a_off: the item's first routed row modulo 4 (the offset of the MX activation code planes)
template <class C, bool B_KN, class O>
MI355_HD void read_frags(Frags<C::MX, B_KN, C::MI>& f, const uint8_t* slot, int h, int rbo, int wq, int lane_in,
                         int a_off, int nmi) {
  constexpr bool MX = C::MX;
  constexpr int MI = C::MI;
  // bf16 tiles of five row blocks: the fragment addresses are recomputed per read (held across the
  // K loop they would take about 28 registers)
  const int lane = (!MX && MI > 4) ? O::opaque(lane_in) : lane_in;
  const uint8_t* As = slot;
  const uint8_t* Bs = slot + C::B_OFF;
  if constexpr (!MX) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int ks = h * 2 + s2;  // 16-K step of the stage
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        if (MI > 4 && mi >= nmi) continue;  // row block without rows of the item
        const int r = (C::RBS * mi + rbo) * 32 + (lane & 31);
        f.a[s2][mi] = O::template lds<v8bf>(As + chunk_off(r, ks * 2 + (lane >> 5)));
      }
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        if constexpr (!B_KN) {
          const int n = wq * WN + ni * 32 + (lane & 31);
          f.b[s2][ni] = O::template lds<v8bf>(Bs + chunk_off(n, ks * 2 + (lane >> 5)));
        } else {
          const int g16 = lane >> 4, m = lane & 15;
          const int nb = wq * WN + ni * 32 + (g16 & 1) * 16 + 4 * (m & 3);
          const int k0 = ks * 16 + (g16 >> 1) * 8 + (m >> 2), k1 = k0 + 4;
          const int off0 = k0 * (2 * C::BN) + (((nb >> 3) ^ ((k0 & 7) << 1)) << 4) + (nb & 7) * 2;
          const int off1 = k1 * (2 * C::BN) + (((nb >> 3) ^ ((k1 & 7) << 1)) << 4) + (nb & 7) * 2;
          f.bl[s2][ni] = O::tr16(Bs + off0);
          f.bh[s2][ni] = O::tr16(Bs + off1);
        }
      }
    }
  } else {
    // one 64-K step h: lane r + 32 g holds K 16 g .. +15 and 32 + 16 g .. +15 of the step
    const uint8_t* ASs = slot + C::AS_OFF;
    const uint8_t* BSs = slot + C::BS_OFF;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const int r = (C::RBS * mi + rbo) * 32 + (lane & 31);
      const int c0 = h * 4 + (lane >> 5);
      f.al[mi] = O::template lds<v4i>(As + chunk_off(r, c0));
      f.ah[mi] = O::template lds<v4i>(As + chunk_off(r, c0 + 2));
      f.sa[mi] = O::template lds<uint8_t>(ASs + (h * 2 + (lane >> 5)) * AS_PLANE + a_off + r);
    }
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int n = wq * WN + ni * 32 + (lane & 31);
      if constexpr (!B_KN) {
        const int c0 = h * 4 + (lane >> 5);
        f.bl[ni] = O::template lds<v4i>(Bs + chunk_off(n, c0));
        f.bh[ni] = O::template lds<v4i>(Bs + chunk_off(n, c0 + 2));
      } else {
        const int g16 = lane >> 4, m = lane & 15;
        const int nb = wq * WN + ni * 32 + (g16 & 1) * 16;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int k = h * 64 + (q >> 1) * 32 + (g16 >> 1) * 16 + (q & 1) * 8 + (m >> 1);
          constexpr int M = (1 << C::B_CH_LOG) - 1;
          const int off = k * C::BN + (((nb >> 4) ^ (k & M)) << 4) + 8 * (m & 1);
          f.bp[ni][q] = O::tr8(Bs + off);
        }
      }
      f.sb[ni] = O::template lds<uint8_t>(BSs + h * (2 * C::BN) + n * 2 + (lane >> 5));
    }
  }
}

// nmi: the wave's row blocks that hold rows of the item (bf16 320-row tiles skip the others, so a
// tile of up to 256 rows issues the MFMAs a 256-row tile would)
template <bool MX, bool B_KN, int MI, class O>
MI355_HD void mfmas(const Frags<MX, B_KN, MI>& f, v16f (&acc)[MI][NI], int nmi) {
  if constexpr (!MX) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          if (MI > 4 && mi >= nmi) continue;
          v8bf b;
          if constexpr (!B_KN) b = f.b[s2][ni];
          else b = __builtin_bit_cast(v8bf, __builtin_shufflevector(f.bl[s2][ni], f.bh[s2][ni], 0, 1, 2, 3, 4, 5, 6, 7));
          O::mfma_bf16(f.a[s2][mi], b, acc[mi][ni]);
        }
  } else {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const v8i a = __builtin_shufflevector(f.al[mi], f.ah[mi], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        v8i b;
        if constexpr (!B_KN) {
          b = __builtin_shufflevector(f.bl[ni], f.bh[ni], 0, 1, 2, 3, 4, 5, 6, 7);
        } else {
          const v4i b01 = __builtin_shufflevector(f.bp[ni][0], f.bp[ni][1], 0, 1, 2, 3);
          const v4i b23 = __builtin_shufflevector(f.bp[ni][2], f.bp[ni][3], 0, 1, 2, 3);
          b = __builtin_shufflevector(b01, b23, 0, 1, 2, 3, 4, 5, 6, 7);
        }
        O::mfma_f8(a, b, acc[mi][ni], f.sa[mi], f.sb[ni]);
      }
    }
  }
}

template <class O>
MI355_HD float swiglu_act(float g_acc, float u_acc) {
  // the gate and up projections are rounded to bf16 (the GMM1 output), SiLU(gate) * up in fp32
  const float gte = bf16_to_f32(f32_to_bf16(g_acc));
  const float up = bf16_to_f32(f32_to_bf16(u_acc));
  return gte / (1.0f + O::expf(-gte)) * up;
}

// Staging offset of element (row, byte column cb) of a 32 x 64-byte block: 16-byte chunks swizzled
// with (row >> 2) & 3, so the two half-wavefronts (rows r and r + 4) write different banks.
MI355_HD int stage_off(int row, int cb) { return row * 64 + ((((cb >> 4) ^ (row >> 2)) & 3) << 4) + (cb & 15); }

// acc[mi][ni][r] holds row (RBS mi + rbo) * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4 and column
// wq * 64 + ni * 32 + lane % 32 of the tile. Each 32 x 32 output block goes through the wave's LDS
// staging block 16 rows at a time (LDS operations of a wave complete in order) and is written with
// 16-byte stores (fp32: 32 bytes, MX: 8 e4m3 bytes per lane and the block's scale code).
template <class C, int EPI, class O>
MI355_HD void epilogue(const GGParams& p, const Item& it, const v16f (&acc)[C::MI][NI], int rbo, int wq, int lane_in,
                       uint8_t* stage) {
  constexpr int MI = C::MI;
  // the lane index made opaque: the staging offsets are recomputed here instead of being hoisted out
  // of the K loop (where they would take registers for the whole loop)
  const int lane = O::opaque(lane_in);
  const typename O::lds_ptr st = O::lds_base(stage);
  constexpr int NB = EPI == EPI_STORE_BF16 ? NI : 1;  // output blocks per 32 rows
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    const int row_base = (C::RBS * mi + rbo) * 32;  // first tile row of the block
    if (row_base >= it.rows) continue;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (EPI == EPI_SWIGLU_F32 || EPI == EPI_SWIGLU_MX) {
        // Two halves of 16 rows: the fp32 SwiGLU values go through the staging block (16 rows x 128
        // bytes); lane l then holds row l / 4, columns 8 (l % 4) ..+7 of the 32-column block cb of the
        // output rows.
        const int cb = it.nt * (C::BN / 64) + wq;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int r = 8 * hh; r < 8 * hh + 8; ++r) {
            const int lrow = 8 * ((r >> 2) & 1) + 4 * (lane >> 5) + (r & 3);  // row within the half
            const float act = swiglu_act<O>(acc[mi][0][r], acc[mi][1][r]);
            O::template lds_store<float>(st + lrow * 128 + ((((lane & 31) >> 2) ^ (lrow & 7)) << 4) + (lane & 3) * 4,
                                         act);
          }
          const int lrow = lane >> 2, part = lane & 3;
          const v4f v0 = O::template lds_load<v4f>(st + lrow * 128 + (((2 * part) ^ (lrow & 7)) << 4));
          const v4f v1 = O::template lds_load<v4f>(st + lrow * 128 + (((2 * part + 1) ^ (lrow & 7)) << 4));
          const int row = hh * 16 + lrow;
          if constexpr (EPI == EPI_SWIGLU_MX) {
            // MX requantisation of the row's 32-column block: the 4 lanes of a row hold its 32 values
            float amax = fmaxf(fmaxf(fmaxf(fabsf(v0[0]), fabsf(v0[1])), fmaxf(fabsf(v0[2]), fabsf(v0[3]))),
                               fmaxf(fmaxf(fabsf(v1[0]), fabsf(v1[1])), fmaxf(fabsf(v1[2]), fabsf(v1[3]))));
            amax = fmaxf(amax, O::shfl_xor(amax, 1));
            amax = fmaxf(amax, O::shfl_xor(amax, 2));
            const uint32_t code = mx_scale_code(amax);
            v2i w;
            w[0] = (int)(O::e4m3(mx_apply_inv_scale(v0[0], code)) | (O::e4m3(mx_apply_inv_scale(v0[1], code)) << 8) |
                         (O::e4m3(mx_apply_inv_scale(v0[2], code)) << 16) |
                         (O::e4m3(mx_apply_inv_scale(v0[3], code)) << 24));
            w[1] = (int)(O::e4m3(mx_apply_inv_scale(v1[0], code)) | (O::e4m3(mx_apply_inv_scale(v1[1], code)) << 8) |
                         (O::e4m3(mx_apply_inv_scale(v1[2], code)) << 16) |
                         (O::e4m3(mx_apply_inv_scale(v1[3], code)) << 24));
            if (row_base + row < it.rows) {
              const int64_t orow = it.row0 + row_base + row;
              O::template store<v2i>((uint8_t*)p.C + orow * p.ldc + cb * 32 + part * 8, w);
              if (part == 0)  // the code of block cb: plane cb % 4 of the 128-column stage cb / 4
                O::template store<uint8_t>(
                    p.c_scale + (cb >> 2) * p.c_scale_stage_stride + (cb & 3) * (p.c_scale_stage_stride >> 2) + orow,
                    (uint8_t)code);
            }
          } else if (row_base + row < it.rows) {
            float* dst = (float*)p.C + (it.row0 + row_base + row) * p.ldc + cb * 32 + part * 8;
            O::template store<v4f>(dst, v0);
            O::template store<v4f>(dst + 4, v1);
          }
        }
      } else {
        // two halves of 16 rows: bf16 values into the staging block (16 rows x 64 bytes), then
        // 16 bytes per lane (row lane / 4, columns 8 (lane % 4) ..+7) out
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int r = 8 * hh; r < 8 * hh + 8; ++r) {
            const int row = 8 * ((r >> 2) & 1) + 4 * (lane >> 5) + (r & 3);  // row within the half
            float v;
            if constexpr (EPI == EPI_STORE_BF16) v = acc[mi][nb][r];
            else v = swiglu_act<O>(acc[mi][0][r], acc[mi][1][r]);
            const uint16_t hv = f32_to_bf16(v);  // (the value before the address, as an assignment orders them)
            O::template lds_store<uint16_t>(st + stage_off(row, (lane & 31) * 2), hv);
          }
          const int row = lane >> 2, c = lane & 3;
          const v4i v = O::template lds_load<v4i>(st + stage_off(row, c * 16));
          const int col = EPI == EPI_STORE_BF16 ? it.nt * C::BN + wq * WN + nb * 32 + c * 8
                                                : it.nt * (C::BN / 2) + wq * 32 + c * 8;
          if (row_base + hh * 16 + row < it.rows && col < p.N) {
            const int64_t orow = it.row0 + row_base + hh * 16 + row;
            O::template store<v4i>((uint16_t*)p.C + orow * p.ldc + col, v);
          }
        }
      }
    }
  }
}

// ---- configuration of a call (host) -------------------------------------------------------------
// 320-row tiles for bf16 when the caller's row count averages at most 320 per group
inline bool pp_tall(const GGParams& p, bool mx) {
  return !mx && p.rows_hint > 0 && p.rows_hint <= (int64_t)p.G * 320 && p.G <= Cfg<false, true>::PREFIX_MAX;
}

// The skinny tile for the groups above the other tile's height and up to 384 rows, when switched on
// and the rows average 128..512 per group (else few groups fall in the range)
inline bool pp_skinny(const GGParams& p) {
  return mi355_pp_skinny_enabled() && p.G <= Cfg<true, false, true>::PREFIX_MAX &&
         p.rows_hint >= (int64_t)p.G * 128 && p.rows_hint <= (int64_t)p.G * 512;
}

// The regular launch over the groups outside the skinny range (tile height from TALL), then the
// skinny one over the rest, whose n-tiles are half as wide.
template <bool MX, bool B_KN, int EPI, bool TALL, class Launch>
int pp_run_skinny(const GGParams& p, Launch& L) {
  const int rc = L.template run<MX, B_KN, EPI, TALL, SEL_NOT_SKINNY>(p);
  if (rc) return rc;
  GGParams q = p;
  constexpr int cols = EPI == EPI_STORE_BF16 ? Cfg<MX, false, true>::BN : Cfg<MX, false, true>::BN / 2;
  q.n_tiles = (p.N + cols - 1) / cols;
  return L.template run<MX, B_KN, EPI, false, Cfg<MX, TALL>::BM == 320 ? SEL_SKINNY_320 : SEL_SKINNY_256>(q);
}

// The kernel instances of a call that mi355_gg_pp_applies accepted: L.template run<MX, B_KN, EPI,
// TALL, SEL>(p), one launch, or two with the skinny tile. The library launches them; the host-side
// checker replays them.
template <bool MX, bool B_KN, int EPI, class Launch>
int pp_select_tall(const GGParams& p, Launch& L) {
  if constexpr (!MX) {
    const bool tall = pp_tall(p, MX);
    if (pp_skinny(p))
      return tall ? pp_run_skinny<MX, B_KN, EPI, true>(p, L) : pp_run_skinny<MX, B_KN, EPI, false>(p, L);
    if (tall) return L.template run<MX, B_KN, EPI, true, SEL_ALL>(p);
  } else {
    if (pp_skinny(p)) return pp_run_skinny<MX, B_KN, EPI, false>(p, L);
  }
  return L.template run<MX, B_KN, EPI, false, SEL_ALL>(p);
}
template <class Launch>
int pp_select(const GGParams& p, bool mx, bool b_kn, int epi, Launch& L) {
  if (!mx) {
    if (!b_kn) return epi == EPI_STORE_BF16 ? pp_select_tall<false, false, EPI_STORE_BF16>(p, L)
                                            : pp_select_tall<false, false, EPI_SWIGLU_BF16>(p, L);
    return epi == EPI_STORE_BF16 ? pp_select_tall<false, true, EPI_STORE_BF16>(p, L)
                                 : pp_select_tall<false, true, EPI_SWIGLU_BF16>(p, L);
  }
  return epi == EPI_STORE_BF16 ? pp_select_tall<true, true, EPI_STORE_BF16>(p, L)
                               : pp_select_tall<true, true, EPI_SWIGLU_F32>(p, L);
}

}  // namespace pp
