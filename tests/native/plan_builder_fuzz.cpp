// Host-only fuzz of the plan builder under AddressSanitizer: random (valid and invalid)
// segment tables through emrs_plan_create / stats / destroy, plus tuning calls.
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <random>
#include <vector>
#include "emrs.h"

int main(int argc, char **argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 2000;
  std::mt19937_64 rng(12345);
  auto U = [&](uint64_t lo, uint64_t hi) { return lo + rng() % (hi - lo + 1); };
  int ok = 0, bad = 0;
  for (int it = 0; it < iters; ++it) {
    const uint32_t ns = (uint32_t)U(1, 5), nd = (uint32_t)U(1, 5);
    std::vector<uint64_t> sb(ns), db(nd);
    for (auto &x : sb) x = U(1 << 17, 1 << 22);
    for (auto &x : db) x = U(1 << 17, 1 << 22);
    const uint64_t n = U(0, 6);
    std::vector<emrs_segment> t(n);
    for (auto &s : t) {
      memset(&s, 0, sizeof s);
      const uint32_t ebs[4] = {1, 2, 4, 8};
      s.elem_bytes = rng() % 23 == 0 ? (uint32_t)U(0, 9) : ebs[rng() % 4];
      s.src_buf = (uint32_t)(rng() % 30 ? U(0, ns - 1) : U(0, ns));  // sometimes out of range
      s.dst_buf = (uint32_t)(rng() % 30 ? U(0, nd - 1) : U(0, nd));
      s.rows = rng() % 3 ? 1 : U(1, 40);
      s.len = U(0, 600);
      s.src_stride = s.rows > 1 ? s.len + U(0, 50) - (rng() % 10 == 0 ? 60 : 0) : 0;
      s.dst_stride = s.rows > 1 ? s.len + U(0, 50) : 0;
      s.src_off = U(0, 1 << 12);
      s.dst_off = U(0, 1 << 12);
      const int kind = rng() % 6;
      if (kind == 0 && s.elem_bytes == 4) { s.flags = EMRS_SEG_CAST_BF16; s.aux_buf = (uint32_t)U(0, nd - 1); s.aux_off = U(0, 1 << 12); s.aux_stride = s.rows > 1 ? s.len + U(0, 9) : 0; }
      if (kind == 1) { s.flags = EMRS_SEG_DUP; s.aux_buf = (uint32_t)U(0, nd - 1); s.aux_off = U(0, 1 << 12); s.aux_stride = s.rows > 1 ? s.len + U(0, 9) : 0; }
      if (kind == 2) s.flags |= EMRS_SEG_ZERO_FILL;
      if (rng() % 50 == 0) s.flags |= 0x80;  // unknown flag
      if (rng() % 50 == 0) s.reserved = 1;
      if (rng() % 40 == 0) { s.src_off = ~0ull - U(0, 100); }  // overflow
      if (rng() % 40 == 0) { s.len = (1ull << 31) + U(0, 10); }
    }
    emrs_plan *p = nullptr;
    const uint32_t flags = rng() % 2 ? EMRS_PLAN_CHECK_DISJOINT : 0;
    int rc = emrs_plan_create(t.data(), n, sb.data(), ns, db.data(), nd, flags, &p);
    if (rc == EMRS_OK) {
      ++ok;
      emrs_plan_stats st;
      if (emrs_plan_stats_get(p, &st) != EMRS_OK) { fprintf(stderr, "stats failed\n"); return 1; }
      std::vector<void *> s(ns, (void *)0x1000), d(nd, (void *)0x100000);
      (void)emrs_plan_execute(p, s.data(), d.data(), nullptr);  // no device: must refuse
      (void)emrs_plan_prepare(p, nullptr);                       // likewise
      emrs_plan_destroy(p);
    } else {
      ++bad;
      if (p) { fprintf(stderr, "plan set on failure\n"); return 1; }
      if (!emrs_last_error()[0]) { fprintf(stderr, "no message for rc %d\n", rc); return 1; }
    }
  }
  emrs_tuning tu;
  for (int i = 0; i < 200; ++i) {
    emrs_get_tuning(&tu);
    tu.lanes = (uint32_t)U(0, 300); tu.units = (uint32_t)U(0, 5); tu.xcd_remap = (uint32_t)U(0, 3);
    tu.warm_tables = (uint32_t)U(0, 2);
    (void)emrs_set_tuning(&tu);
  }
  // Hand-off records refused on the host, before any driver call: allocations of 2 GiB or more,
  // buffers past their allocation, misaligned offsets, a set reserved field; unknown pointers.
  for (int i = 0; i < 2000; ++i) {
    emrs_ipc_buffer b;
    memset(&b, 0, sizeof b);
    for (auto &x : b.handle) x = (uint8_t)rng();
    const int kind = (int)(rng() % 4);
    b.allocation_bytes = kind == 0 ? EMRS_IPC_MAX_ALLOCATION_BYTES + U(0, 1ull << 40) : U(1, 1ull << 30);
    b.offset = kind == 2 ? U(0, 15) | 1 : U(0, b.allocation_bytes) & ~15ull;
    b.bytes = kind == 1 ? b.allocation_bytes - std::min(b.offset, b.allocation_bytes) + U(1, 100) : 0;
    b.reserved = kind == 3 ? (uint32_t)U(1, 9) : 0;
    void *ptr = (void *)0x1;
    const int rc = emrs_ipc_open(&b, &ptr);
    if (rc == EMRS_OK || ptr != nullptr || !emrs_last_error()[0]) {
      fprintf(stderr, "ipc record %d (kind %d) not refused: rc %d\n", i, kind, rc);
      return 1;
    }
    if (emrs_ipc_close((void *)(uintptr_t)U(1, 1ull << 48)) == EMRS_OK) {
      fprintf(stderr, "close of an unknown pointer accepted\n");
      return 1;
    }
  }
  if (emrs_ipc_open_count() != 0 || emrs_ipc_open(nullptr, nullptr) == EMRS_OK ||
      emrs_ipc_export(nullptr, 16, nullptr) == EMRS_OK) {
    fprintf(stderr, "ipc argument checks\n");
    return 1;
  }
  printf("ok %d rejected %d\n", ok, bad);
  return 0;
}
