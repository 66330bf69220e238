// Runs the one-launch decode prologue (decode_prep.h) under the host emulation of prep_sim.inc on
// inputs from a file and writes its outputs to another (test infrastructure; tests/test_decode_prep.py
// compares them with the oracle).
//
//   prep_check IN OUT [MUTATION]
// IN:  int64 header {i64 ids, slots, E, bm, rows, cols, flags} (flags: 1 counts, 2 group_list,
//      4 gather, 8 error_flag, 16 tile_prefix), then the ids (int32 or int64), then x [rows, cols]
//      bf16.
// OUT: int64 {ballots, workgroups}, counts [E] i32, group_list [E] i64, mapping [slots] i32, gather
//      [slots] i32, error_flag i32, tile_prefix [E + 1] i32, q [rows, cols] u8, scale [rows, cols/32]
//      u8 (absent outputs as their fill value: -7 for int32 / int64 buffers, 0x5a for bytes).
// Every output buffer is an allocation of its exact size, so the AddressSanitizer build reports any
// access past it.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "prep_sim.inc"

static std::vector<uint8_t> slurp(const char* path) {
  FILE* f = fopen(path, "rb");
  if (!f) {
    perror(path);
    exit(2);
  }
  std::vector<uint8_t> b;
  uint8_t buf[1 << 16];
  size_t n;
  while ((n = fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + n);
  fclose(f);
  return b;
}

template <class T>
static T* alloc(int64_t n, int fill) {
  T* p = (T*)malloc((size_t)(n > 0 ? n : 1) * sizeof(T));
  memset(p, fill, (size_t)(n > 0 ? n : 1) * sizeof(T));
  return p;
}

int main(int argc, char** argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: prep_check IN OUT [MUTATION]\n");
    return 2;
  }
  const int mutation = argc > 3 ? atoi(argv[3]) : 0;
  std::vector<uint8_t> in = slurp(argv[1]);
  int64_t h[7];
  if (in.size() < sizeof h) return 2;
  memcpy(h, in.data(), sizeof h);
  const bool i64 = h[0] != 0;
  const int64_t slots = h[1], rows = h[4];
  const int E = (int)h[2], bm = (int)h[3], cols = (int)h[5], flags = (int)h[6];
  const size_t id_bytes = (size_t)slots * (i64 ? 8 : 4), x_bytes = (size_t)(rows * cols * 2);
  if (in.size() != sizeof h + id_bytes + x_bytes) {
    fprintf(stderr, "input size %zu, expected %zu\n", in.size(), sizeof h + id_bytes + x_bytes);
    return 2;
  }
  void* ids = malloc(id_bytes ? id_bytes : 1);
  memcpy(ids, in.data() + sizeof h, id_bytes);
  uint16_t* x = alloc<uint16_t>(rows * cols, 0);
  memcpy(x, in.data() + sizeof h + id_bytes, x_bytes);
  const int nb = cols / 32;
  dprep::Args a = {};
  a.ids = ids;
  a.slots = slots;
  a.E = E;
  a.bm = bm;
  int32_t* counts = alloc<int32_t>(E, 0xf9);
  int64_t* group_list = alloc<int64_t>(E, 0xf9);
  int32_t* mapping = alloc<int32_t>(slots, 0xf9);
  int32_t* gather = alloc<int32_t>(slots, 0xf9);
  int32_t* err = alloc<int32_t>(1, 0);
  int32_t* tile_prefix = alloc<int32_t>(E + 1, 0xf9);
  uint8_t* q = alloc<uint8_t>(rows * cols, 0x5a);
  uint8_t* scale = alloc<uint8_t>(rows * nb, 0x5a);
  a.counts = flags & 1 ? counts : nullptr;
  a.group_list = flags & 2 ? group_list : nullptr;
  a.mapping = mapping;
  a.gather = flags & 4 ? gather : nullptr;
  a.error_flag = flags & 8 ? err : nullptr;
  a.tile_prefix = flags & 16 ? tile_prefix : nullptr;
  a.x = x;
  a.rows = rows;
  a.cols = cols;
  a.q = q;
  a.scale = scale;
  a.scale_ld = nb;
  auto release = [&] {
    free(ids), free(x), free(counts), free(group_list), free(mapping), free(gather), free(err), free(tile_prefix);
    free(q), free(scale);
  };
  prep_sim::Stats st;
  if (prep_sim::run(a, i64, mutation, &st) != 0) {
    fprintf(stderr, "arguments refused\n");
    release();
    return 3;
  }
  FILE* f = fopen(argv[2], "wb");
  if (!f) {
    release();
    return 2;
  }
  const int64_t head[2] = {st.ballots, st.workgroups};
  fwrite(head, sizeof head, 1, f);
  fwrite(counts, 4, E, f);
  fwrite(group_list, 8, E, f);
  fwrite(mapping, 4, slots, f);
  fwrite(gather, 4, slots, f);
  fwrite(err, 4, 1, f);
  fwrite(tile_prefix, 4, E + 1, f);
  fwrite(q, 1, rows * cols, f);
  fwrite(scale, 1, rows * nb, f);
  fclose(f);
  release();
  return 0;
}
