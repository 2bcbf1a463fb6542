// Copy-plan executor for the reshard repack on MI355X (gfx950, CDNA4).
//
// One launch moves every segment of a plan.  The path is pure data movement
// (no arithmetic), so the kernel is shaped for HBM streaming: the plan is cut
// into chunks of 256 units (4 KB of 16-byte units), and every chunk is a
// workgroup of its own, one wave of 64 lanes with four units each, that finds
// its segment by one binary search, issues its four loads, stores and exits.
// The hardware dispatches workgroups in order, so the in-flight ones always
// cover one narrow window of the plan that sweeps through memory; a
// persistent grid, whose workgroups drift apart, writes up to 20% slower on
// most physical placements of the same buffers.  The persistent grid remains
// as a tuning option.  Element sizes are irrelevant to the vector path:
// offsets are converted to 16-byte units when the plan is created, so bf16
// parameters and fp32 optimizer state share one launch.
//
// The reference performs the same movement as per-parameter slicing plus
// point-to-point messages (elastic_megatron/transfer/transfer.py:36-101,
// :143-269; elastic_megatron/transfer/communicator.py:61-96).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <type_traits>
#include <vector>

#include "emrs.h"
#include "internal.h"

namespace {
thread_local std::string g_last_error;
}  // namespace

// Device scratch of emrs_plan_compare_static, the entry point that allocates
// nothing: its accumulators, group ids, segment table and pointer table.  Each
// device holds its own copy for the life of the process; host code reaches it
// only through the address hipGetSymbolAddress returns on that device.
static __device__ __align__(256) unsigned char scratch[EMRS_STATIC_SCRATCH_BYTES];

namespace emrs_internal {
int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}
void clear_error() { g_last_error.clear(); }
}  // namespace emrs_internal

namespace {

using emrs_internal::fail;

int hip_fail(hipError_t e, const char *what) {
  return fail(EMRS_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// A call that has to allocate device memory or upload a table cannot be
// recorded into a HIP graph: the captured copy would read host memory that is
// gone when the graph replays, and the allocation would not be replayed at
// all.  Such calls are refused while `st` is capturing; the caller runs the
// same call once outside the capture first, after which calls with the same
// base pointers need neither.
int refuse_capture(hipStream_t st, const char *what) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  if (cs != hipStreamCaptureStatusNone)
    return fail(EMRS_ERR_CAPTURE, std::string(what) +
                                      " would allocate or upload while the stream is capturing a graph; "
                                      "run the call once before the capture, with the same base pointers");
  return EMRS_OK;
}

#ifndef EMRS_COPY_THREADS
#define EMRS_COPY_THREADS 256  // lanes per workgroup
#endif
#ifndef EMRS_COPY_UNROLL
#define EMRS_COPY_UNROLL 8  // chunks of one segment per step of the persistent and compare kernels
#endif
constexpr int kThreads = EMRS_COPY_THREADS;
constexpr int kUnroll = EMRS_COPY_UNROLL;
constexpr uint32_t kChunkUnits = kThreads;  // units per work chunk: one per lane
constexpr uint32_t kStepUnits = kThreads * kUnroll;  // units per step of a persistent workgroup
constexpr uint64_t kMaxGridY = 65535;                     // rows of a one-workgroup-per-chunk grid
// Plans of at least this many chunks (2 GiB of 16-byte units) give each XCD
// its own contiguous eighth by default.  Measured on Llama-2-7B-shaped
// switches: at 0.69M chunks and up it saved 0.3-2%; at 0.11M and 0.24M chunks
// it cost 5.8% and 1.4%, the launch being too short for per-XCD windows.
constexpr uint64_t kXcdRemapMinChunks = 1ull << 19;
constexpr uint64_t kMaxUnitsPerSeg = 1ull << 30;       // keeps unit math in 32 bits
constexpr int kDifferBlocksPerCu = 4;                  // workgroups per CU of a comparison's first pass
// Row pitches of multi-row segments stay below this many bytes, so that a piece
// of at most 256 rows spans less than 2^31 bytes from its first row: the
// buffer-instruction path addresses it with 32-bit offsets.  Segments with
// longer pitches are emitted one row at a time.
constexpr uint64_t kMaxPitchBytes = 1ull << 23;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Buffers passed by value in kernel arguments; plans with more buffers on
// either side pass a device-memory table of pointers instead.  (Kernel
// arguments are limited to a few KB: this table must stay small.)
constexpr uint32_t kArgBuffers = 128;

struct Bases {
  char *p[kArgBuffers];
};
static_assert(sizeof(Bases) <= 1024, "Bases travels in kernel arguments");

// Where a chunk's segment search starts and ends: chunk c lies in one of the
// segments first[c >> shift] .. first[(c >> shift) + 1], so the search spans
// a few dozen segments of the plan instead of all of them.  Travels in
// kernel arguments beside the two Bases.
constexpr uint32_t kHintBuckets = 256;
struct SegHint {
  uint32_t first[kHintBuckets + 1];
  uint32_t shift;
};
static_assert(2 * sizeof(Bases) + sizeof(SegHint) + 64 <= 4096, "kernel arguments stay under 4 KB");

// Segment as the kernel sees it.  Offsets and strides are in units of
// (1 << unit_log2) bytes: 16 for the vector path, the element size otherwise.
// A cast segment (fp32 only) also writes bf16 copies to aux, whose offset and
// stride are in units of half that size (8 bytes, or one bf16).  A duplicating
// segment writes its values to aux as well, in the segment's own units.
struct DevSeg {
  uint64_t src_off;
  uint64_t dst_off;
  uint64_t chunk_begin;  // index of this segment's first chunk
  uint64_t aux_off;
  uint32_t len;          // units per row
  uint32_t rows;
  uint32_t src_stride;
  uint32_t dst_stride;
  uint32_t aux_stride;
  uint32_t magic;        // row = (t + ((u - t) >> sh1)) >> sh2, t = umulhi(magic, u)
  // Whole 32-bit words only, so that a workgroup reads its descriptor with
  // scalar loads alone (the compiler reads 8- and 16-bit fields with vector
  // loads, which put a vector-memory round trip ahead of the workgroup's data).
  uint32_t bufs;         // bits 0-15: source buffer; bits 16-31: destination buffer
  uint32_t meta;         // bits 0-15: second destination (aux) buffer; 16-23: shifts; 24-31: kind

  // shifts: bits 0-4 sh2, bit 5 sh1.  kind: bits 0-2 unit_log2, bits 3-4
  // elem_log2, bits 5-7 ops.  ops bit 0: also write bf16 to aux; bit 1: write
  // zeros, read nothing; bit 2: also write the values unchanged to aux.
  // elem_log2: element size of the input segment (read by the compare kernel
  // and for duplicates).
  __host__ __device__ uint32_t src_buf() const { return bufs & 0xffffu; }
  __host__ __device__ uint32_t dst_buf() const { return bufs >> 16; }
  __host__ __device__ uint32_t aux_buf() const { return meta & 0xffffu; }
  __host__ __device__ uint32_t sh1() const { return (meta >> 21) & 1u; }
  __host__ __device__ uint32_t sh2() const { return (meta >> 16) & 31u; }
  __host__ __device__ uint32_t unit_log2() const { return (meta >> 24) & 7u; }
  __host__ __device__ uint32_t elem_log2() const { return (meta >> 27) & 3u; }
  __host__ __device__ uint32_t ops() const { return meta >> 29; }
  void set_bufs(uint32_t src, uint32_t dst, uint32_t aux) {
    bufs = (src & 0xffffu) | (dst << 16);
    meta = (meta & 0xffff0000u) | (aux & 0xffffu);
  }
  void set_kind(uint32_t sh2_, uint32_t sh1_, uint32_t unit_log2_, uint32_t elem_log2_, uint32_t ops_) {
    meta = (meta & 0xffffu) | ((sh2_ | (sh1_ << 5)) << 16) | ((unit_log2_ | (elem_log2_ << 3) | (ops_ << 5)) << 24);
  }
};
static_assert(sizeof(DevSeg) == 64, "DevSeg layout");

// Division by an invariant divisor (Granlund & Montgomery 1994, fig. 4.1).
void make_magic(uint32_t d, uint32_t *m, uint32_t *sh1, uint32_t *sh2) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  uint64_t num = (uint64_t)(((unsigned __int128)1 << 32) * (((unsigned __int128)1 << l) - d) / d) + 1;
  *m = (uint32_t)num;
  *sh1 = l < 1 ? l : 1;
  *sh2 = l > 1 ? l - 1 : 0;
}

__host__ __device__ __forceinline__ uint32_t umulhi32(uint32_t a, uint32_t b) {
  return (uint32_t)(((uint64_t)a * b) >> 32);
}

__host__ __device__ __forceinline__ uint32_t magic_div(uint32_t n, uint32_t m, uint32_t sh1,
                                                       uint32_t sh2) {
  uint32_t t = umulhi32(m, n);
  return (t + ((n - t) >> sh1)) >> sh2;
}

struct Tuning {
  std::atomic<uint32_t> blocks_per_cu{0};  // persistent grid: 0 = as many as can be resident
  std::atomic<uint32_t> nontemporal{1};
  std::atomic<uint32_t> xcd_remap{1};      // 0, 1 (by plan size) or 2
  std::atomic<uint32_t> run{4};            // persistent grid: round-robin runs of 4 x kUnroll chunks
  std::atomic<uint32_t> persistent{0};     // 0: one workgroup per piece of a chunk
  std::atomic<uint32_t> lanes{64};         // lanes per workgroup of one piece: 64, 128 or 256
  std::atomic<uint32_t> units{1};          // 16-byte units per lane: lanes * units is 64, 128 or 256
  std::atomic<uint32_t> buffer_ops{0};     // 1: 16-byte units through buffer instructions
  std::atomic<uint32_t> chunk_index{1};    // 1: each chunk's segment from the plan's chunk table
  std::atomic<uint32_t> warm_tables{1};    // 1: read the chunk and segment tables just before the copy
};
Tuning g_tuning;

// ---------------------------------------------------------------------------
// Copy kernel
// ---------------------------------------------------------------------------

template <typename T, bool kNT>
__device__ __forceinline__ T ld(const T *p) {
  if constexpr (kNT) return __builtin_nontemporal_load(p);
  else return *p;
}

template <typename T, bool kNT>
__device__ __forceinline__ void st(T *p, T v) {
  if constexpr (kNT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// fp32 -> bf16 rounded to nearest even; NaN becomes the quiet NaN 0x7FC0
// (the rounding torch applies in float -> bfloat16 conversions).
__device__ __forceinline__ uint32_t bf16_rne(uint32_t u) {
  return (u & 0x7fffffffu) > 0x7f800000u ? 0x7fc0u : (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

template <typename T>
struct CastOf;  // bf16 image of one unit
template <>
struct CastOf<u32x4> {
  typedef unsigned int type __attribute__((ext_vector_type(2)));
  __device__ static type cast(u32x4 v) {
    type r;
    r.x = bf16_rne(v.x) | (bf16_rne(v.y) << 16);
    r.y = bf16_rne(v.z) | (bf16_rne(v.w) << 16);
    return r;
  }
};
template <>
struct CastOf<uint32_t> {
  typedef uint16_t type;
  __device__ static type cast(uint32_t v) { return (uint16_t)bf16_rne(v); }
};

// Copy units [u0, u_end) of segment s, 0 < u_end - u0 <= kStepUnits; with
// kCast also store each unit's bf16 image to aux.  In a partial chunk, lanes
// past the end load the last unit again (in bounds) so that every load is
// unconditional; only their stores are masked off.
template <typename T, bool kNT, bool kCast, bool kZero = false, bool kDup = false>
__device__ __forceinline__ void copy_chunk(const DevSeg &s, const char *sbase, char *dbase, char *abase,
                                           uint32_t u0, uint32_t u_end) {
  typedef typename std::conditional<kCast, CastOf<T>, CastOf<uint32_t>>::type C;
  typedef typename C::type A;
  const T *src = reinterpret_cast<const T *>(sbase);
  T *dst = reinterpret_cast<T *>(dbase);
  A *aux = reinterpret_cast<A *>(abase);
  T *dup = reinterpret_cast<T *>(abase);  // kDup: the second destination, same unit type
  const uint32_t tid = threadIdx.x;
  const uint32_t n = u_end - u0;
  T v[kUnroll];
  if (s.rows == 1) {
    const T *sp = src + s.src_off + u0;
    T *dp = dst + s.dst_off + u0;
    A *ap = aux + s.aux_off + u0;
    T *pp = dup + s.aux_off + u0;
    if constexpr (kZero) {
#pragma unroll
      for (int j = 0; j < kUnroll; ++j) v[j] = T{};
    }
    if (n == kStepUnits) {
#pragma unroll
      for (int j = 0; j < kUnroll; ++j)
        if constexpr (!kZero) v[j] = ld<T, kNT>(sp + j * kThreads + tid);
#pragma unroll
      for (int j = 0; j < kUnroll; ++j) {
        st<T, kNT>(dp + j * kThreads + tid, v[j]);
        if constexpr (kCast) st<A, kNT>(ap + j * kThreads + tid, C::cast(v[j]));
        if constexpr (kDup) st<T, kNT>(pp + j * kThreads + tid, v[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kUnroll; ++j)
        if constexpr (!kZero) v[j] = ld<T, kNT>(sp + min(j * kThreads + tid, n - 1));
#pragma unroll
      for (int j = 0; j < kUnroll; ++j)
        if (j * kThreads + tid < n) {
          st<T, kNT>(dp + j * kThreads + tid, v[j]);
          if constexpr (kCast) st<A, kNT>(ap + j * kThreads + tid, C::cast(v[j]));
          if constexpr (kDup) st<T, kNT>(pp + j * kThreads + tid, v[j]);
        }
    }
    return;
  }
  uint32_t row[kUnroll], col[kUnroll];
#pragma unroll
  for (int j = 0; j < kUnroll; ++j) {
    const uint32_t u = u0 + min(j * kThreads + tid, n - 1);
    row[j] = magic_div(u, s.magic, s.sh1(), s.sh2());
    col[j] = u - row[j] * s.len;
    if constexpr (kZero) v[j] = T{};
    else v[j] = ld<T, kNT>(src + s.src_off + (uint64_t)row[j] * s.src_stride + col[j]);
  }
#pragma unroll
  for (int j = 0; j < kUnroll; ++j)
    if (j * kThreads + tid < n) {
      st<T, kNT>(dst + s.dst_off + (uint64_t)row[j] * s.dst_stride + col[j], v[j]);
      if constexpr (kCast)
        st<A, kNT>(aux + s.aux_off + (uint64_t)row[j] * s.aux_stride + col[j], C::cast(v[j]));
      if constexpr (kDup) st<T, kNT>(dup + s.aux_off + (uint64_t)row[j] * s.aux_stride + col[j], v[j]);
    }
}

// copy_chunk for the unit width of a segment that carries no bf16 image.
template <bool kNT, bool kCast, bool kZero, bool kDup>
__device__ __forceinline__ void dispatch_units(uint32_t ul, const DevSeg &s, const char *sb, char *db, char *ab,
                                               uint32_t u0, uint32_t u_end) {
  switch (ul) {
    case 4: copy_chunk<u32x4, kNT, kCast, kZero, kDup>(s, sb, db, ab, u0, u_end); break;
    case 3: copy_chunk<uint64_t, kNT, kCast, kZero, kDup>(s, sb, db, ab, u0, u_end); break;
    case 2: copy_chunk<uint32_t, kNT, kCast, kZero, kDup>(s, sb, db, ab, u0, u_end); break;
    case 1: copy_chunk<uint16_t, kNT, kCast, kZero, kDup>(s, sb, db, ab, u0, u_end); break;
    default: copy_chunk<uint8_t, kNT, kCast, kZero, kDup>(s, sb, db, ab, u0, u_end); break;
  }
}

// Base address of buffer i: from the kernel-argument table, or (kTable) from
// a device-memory table of pointers for plans with more buffers than fit in
// kernel arguments.
template <bool kTable>
__device__ __forceinline__ char *base_of(const Bases &b, const uint64_t *tab, uint32_t i) {
  if constexpr (kTable) return reinterpret_cast<char *>(tab[i]);
  else return b.p[i];
}

// Copy chunks [c, c_end), starting from the segment that contains chunk c
// (persistent grid).
template <bool kNT, bool kTable>
__device__ __forceinline__ void copy_chunk_run(const DevSeg *__restrict__ segs, uint32_t n_segs, uint64_t n_chunks,
                                               uint64_t c, uint64_t c_end, const Bases &src, const Bases &dst,
                                               const uint64_t *src_tab, const uint64_t *dst_tab) {
  // Last segment whose first chunk is <= c.
  uint32_t lo = 0, hi = n_segs - 1;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (segs[mid].chunk_begin <= c) lo = mid;
    else hi = mid - 1;
  }
  uint32_t si = lo;
  DevSeg s = segs[si];
  uint64_t s_end = (si + 1 < n_segs) ? segs[si + 1].chunk_begin : n_chunks;

  for (uint64_t nq; c < c_end; c += nq) {
    while (c >= s_end) {
      ++si;
      s = segs[si];
      s_end = (si + 1 < n_segs) ? segs[si + 1].chunk_begin : n_chunks;
    }
    // Up to kUnroll chunks of this segment in one step.
    nq = min(min(c_end, s_end) - c, (uint64_t)kUnroll);
    const uint32_t total = s.len * s.rows;
    const uint32_t u0 = (uint32_t)(c - s.chunk_begin) * kChunkUnits;
    const uint32_t u_end = min(u0 + (uint32_t)nq * kChunkUnits, total);
    const char *sb = base_of<kTable>(src, src_tab, s.src_buf());
    char *db = base_of<kTable>(dst, dst_tab, s.dst_buf());
    char *ab = base_of<kTable>(dst, dst_tab, s.aux_buf());
    const uint32_t ops = s.ops(), ul = s.unit_log2();
    if (ops & 4) {  // duplicate to aux, with or without zero fill
      if (ops & 2) dispatch_units<kNT, false, true, true>(ul, s, sb, db, ab, u0, u_end);
      else dispatch_units<kNT, false, false, true>(ul, s, sb, db, ab, u0, u_end);
      continue;
    }
    if (ops & 2) {  // zero fill, with or without the bf16 image
      if (ops & 1) {
        if (ul == 4) copy_chunk<u32x4, kNT, true, true>(s, sb, db, ab, u0, u_end);
        else copy_chunk<uint32_t, kNT, true, true>(s, sb, db, ab, u0, u_end);
      } else {
        dispatch_units<kNT, false, true, false>(ul, s, sb, db, ab, u0, u_end);
      }
      continue;
    }
    if (ops & 1) {
      if (ul == 4) copy_chunk<u32x4, kNT, true>(s, sb, db, ab, u0, u_end);
      else copy_chunk<uint32_t, kNT, true>(s, sb, db, ab, u0, u_end);
      continue;
    }
    dispatch_units<kNT, false, false, false>(ul, s, sb, db, ab, u0, u_end);
  }
}

// Persistent grid (a tuning option).  With run == 0 every workgroup takes one
// contiguous run of chunks_per_block chunks (xcd_stride != 0: each XCD's
// workgroups cover one contiguous slice).  With run > 0 the chunks are dealt
// out round-robin in runs of `run` chunks, so the workgroups sweep the plan
// together; with xcd_stride != 0 as well (the grid is then a multiple of 8,
// and workgroup b runs on XCD b % 8), each XCD sweeps its own contiguous
// eighth, so that no page is touched from two XCDs' translation caches.
template <bool kNT, bool kTable>
__global__ __launch_bounds__(kThreads) void copy_plan_persistent_kernel(
    const DevSeg *__restrict__ segs, uint32_t n_segs, uint64_t n_chunks,
    uint64_t chunks_per_block, uint32_t xcd_stride, uint32_t run, Bases src, Bases dst,
    const uint64_t *__restrict__ src_tab, const uint64_t *__restrict__ dst_tab) {
  if (run) {
    uint64_t c1 = n_chunks, c = (uint64_t)blockIdx.x * run, step = (uint64_t)gridDim.x * run;
    if (xcd_stride) {
      const uint64_t x = blockIdx.x & 7;
      const uint64_t c0 = n_chunks * x / 8;
      c1 = n_chunks * (x + 1) / 8;
      c = c0 + (uint64_t)(blockIdx.x >> 3) * run;
      step = (uint64_t)(gridDim.x >> 3) * run;
    }
    for (; c < c1; c += step)
      copy_chunk_run<kNT, kTable>(segs, n_segs, n_chunks, c, min(c + run, c1), src, dst, src_tab, dst_tab);
    return;
  }
  uint64_t b = blockIdx.x;
  if (xcd_stride) b = (b & 7) * xcd_stride + (b >> 3);  // one contiguous slice per XCD
  const uint64_t c = b * chunks_per_block;
  if (c >= n_chunks) return;
  copy_chunk_run<kNT, kTable>(segs, n_segs, n_chunks, c, min(c + chunks_per_block, n_chunks), src, dst, src_tab,
                              dst_tab);
}

// Units [u0, u0 + L * U) of segment s (clipped to its `total` units) by a
// workgroup of L lanes, U units per lane: every load is issued before the
// first store.
template <typename T, bool kNT, bool kCast, bool kZero, bool kDup, int L, int U>
__device__ __forceinline__ void copy_units(const DevSeg &s, const char *sbase, char *dbase, char *abase, uint32_t u0,
                                           uint32_t total) {
  typedef typename std::conditional<kCast, CastOf<T>, CastOf<uint32_t>>::type C;
  typedef typename C::type A;
  const T *src = reinterpret_cast<const T *>(sbase);
  T *dst = reinterpret_cast<T *>(dbase);
  A *aux = reinterpret_cast<A *>(abase);
  T *dup = reinterpret_cast<T *>(abase);
  T v[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t u = u0 + j * L + threadIdx.x;
    v[j] = T{};
    if constexpr (!kZero) {
      uint64_t so = s.src_off + u;
      if (s.rows > 1) {
        const uint32_t row = magic_div(u, s.magic, s.sh1(), s.sh2());
        so = s.src_off + (uint64_t)row * s.src_stride + (u - row * s.len);
      }
      if (u < total) v[j] = ld<T, kNT>(src + so);
    }
  }
  // Destination offsets are recomputed rather than kept from the loads: with
  // four units per lane that holds the kernel at 66 VGPRs instead of 74, so
  // seven waves fit on each SIMD instead of six.
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t u = u0 + j * L + threadIdx.x;
    if (u < total) {
      uint64_t dof = s.dst_off + u, ao = s.aux_off + u;
      if (s.rows > 1) {
        const uint32_t row = magic_div(u, s.magic, s.sh1(), s.sh2()), col = u - row * s.len;
        dof = s.dst_off + (uint64_t)row * s.dst_stride + col;
        ao = s.aux_off + (uint64_t)row * s.aux_stride + col;
      }
      st<T, kNT>(dst + dof, v[j]);
      if constexpr (kCast) st<A, kNT>(aux + ao, C::cast(v[j]));
      if constexpr (kDup) st<T, kNT>(dup + ao, v[j]);
    }
  }
}

// A buffer resource for raw (unstructured) accesses at 32-bit byte offsets from
// `base`, over the whole 4 GiB range (word 3: the gfx9-family raw-buffer
// configuration).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const char *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(base), 0, -1, 0x00020000);
}

// Cache policy of buffer instructions: bit 1 is the non-temporal hint on gfx94x/gfx950.
template <bool kNT>
struct BufPolicy {
  static constexpr int value = kNT ? 2 : 0;
};

// One unit of T through a buffer instruction at a 32-bit byte offset.
template <typename T, int kPolicy>
__device__ __forceinline__ T buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 16) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kPolicy);
  } else if constexpr (sizeof(T) == 8) {
    const auto w = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kPolicy);
    return (uint64_t)w[0] | ((uint64_t)w[1] << 32);
  } else if constexpr (sizeof(T) == 4) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kPolicy);
  } else if constexpr (sizeof(T) == 2) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kPolicy);
  } else {
    return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, kPolicy);
  }
}

template <typename T, int kPolicy>
__device__ __forceinline__ void buf_store(T v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 16) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kPolicy);
  } else if constexpr (sizeof(T) == 8) {
    typedef unsigned int v2u __attribute__((__vector_size__(8)));
    uint64_t x;
    memcpy(&x, &v, 8);
    const v2u w = {(unsigned)x, (unsigned)(x >> 32)};
    __builtin_amdgcn_raw_buffer_store_b64(w, r, off, 0, kPolicy);
  } else if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kPolicy);
  } else if constexpr (sizeof(T) == 2) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kPolicy);
  } else {
    __builtin_amdgcn_raw_buffer_store_b8(v, r, off, 0, kPolicy);
  }
}

// copy_units with buffer instructions: each stream (source, destination,
// second destination) is one scalar base, the start of the piece's first row,
// plus a 32-bit per-lane byte offset, so a lane needs one VGPR per address
// instead of two.  In a one-row segment the offsets of a lane's units differ
// by constants, which the instructions' immediate offsets hold.  Row pitches
// are below 2^23 bytes (the plan emits longer ones row by row) and a piece
// spans at most 256 rows, so offsets stay below 2^31.  Loads and stores are
// masked exactly as in copy_units.
template <typename T, bool kNT, bool kCast, bool kZero, bool kDup, int L, int U>
__device__ __forceinline__ void copy_units_buf(const DevSeg &s, const char *sbase, char *dbase, char *abase,
                                               uint32_t u0, uint32_t total) {
  typedef typename std::conditional<kCast, CastOf<T>, CastOf<uint32_t>>::type C;
  typedef typename C::type A;
  constexpr int cp = BufPolicy<kNT>::value;
  constexpr uint32_t B = sizeof(T);                          // bytes per unit
  constexpr uint32_t AB = kCast ? sizeof(A) : sizeof(T);     // second-destination bytes per unit
  const uint32_t tid = threadIdx.x;
  T v[U];
  if (s.rows == 1) {
    const __amdgpu_buffer_rsrc_t rs = raw_rsrc(sbase + (s.src_off + u0) * B);
    const __amdgpu_buffer_rsrc_t rd = raw_rsrc(dbase + (s.dst_off + u0) * B);
    const __amdgpu_buffer_rsrc_t ra = raw_rsrc(abase + (s.aux_off + u0) * AB);
    const uint32_t n = total - u0;  // units left in the segment from u0
#pragma unroll
    for (int j = 0; j < U; ++j) {
      v[j] = T{};
      if constexpr (!kZero)
        if (j * L + tid < n) v[j] = buf_load<T, cp>(rs, (j * L + tid) * B);
    }
#pragma unroll
    for (int j = 0; j < U; ++j)
      if (j * L + tid < n) {
        buf_store<T, cp>(v[j], rd, (j * L + tid) * B);
        if constexpr (kCast) buf_store<A, cp>(C::cast(v[j]), ra, (j * L + tid) * AB);
        if constexpr (kDup) buf_store<T, cp>(v[j], ra, (j * L + tid) * AB);
      }
    return;
  }
  const uint32_t row0 = magic_div(u0, s.magic, s.sh1(), s.sh2());
  const __amdgpu_buffer_rsrc_t rs = raw_rsrc(sbase + (s.src_off + (uint64_t)row0 * s.src_stride) * B);
  const __amdgpu_buffer_rsrc_t rd = raw_rsrc(dbase + (s.dst_off + (uint64_t)row0 * s.dst_stride) * B);
  const __amdgpu_buffer_rsrc_t ra = raw_rsrc(abase + (s.aux_off + (uint64_t)row0 * s.aux_stride) * AB);
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t u = u0 + j * L + tid;
    v[j] = T{};
    if constexpr (!kZero)
      if (u < total) {
        const uint32_t row = magic_div(u, s.magic, s.sh1(), s.sh2());
        const uint32_t col = u - row * s.len;
        v[j] = buf_load<T, cp>(rs, ((row - row0) * s.src_stride + col) * B);
      }
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t u = u0 + j * L + tid;
    if (u < total) {
      const uint32_t row = magic_div(u, s.magic, s.sh1(), s.sh2()), dr = row - row0;
      const uint32_t col = u - row * s.len;
      buf_store<T, cp>(v[j], rd, (dr * s.dst_stride + col) * B);
      if constexpr (kCast) buf_store<A, cp>(C::cast(v[j]), ra, (dr * s.aux_stride + col) * AB);
      if constexpr (kDup) buf_store<T, cp>(v[j], ra, (dr * s.aux_stride + col) * AB);
    }
  }
}

template <bool kNT, bool kZero, bool kDup, int L, int U>
__device__ __forceinline__ void dispatch_chunk_buf(uint32_t ul, const DevSeg &s, const char *sb, char *db,
                                                   char *ab, uint32_t u0, uint32_t total) {
  switch (ul) {
    case 4: copy_units_buf<u32x4, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
    case 3: copy_units_buf<uint64_t, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
    case 2: copy_units_buf<uint32_t, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
    case 1: copy_units_buf<uint16_t, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
    default: copy_units_buf<uint8_t, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
  }
}

template <bool kNT, bool kZero, bool kDup, int L, int U>
__device__ __forceinline__ void dispatch_chunk(uint32_t ul, const DevSeg &s, const char *sb, char *db, char *ab,
                                               uint32_t u0, uint32_t total) {
  switch (ul) {
    case 4: copy_units<u32x4, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
    case 3: copy_units<uint64_t, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
    case 2: copy_units<uint32_t, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
    case 1: copy_units<uint16_t, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
    default: copy_units<uint8_t, kNT, false, kZero, kDup, L, U>(s, sb, db, ab, u0, total); break;
  }
}

// One workgroup of L lanes per piece of L * U units of a chunk (the default
// schedule: L = 64, U = 1, four 1 KB pieces per chunk).  A chunk of 256 units
// holds 256 / (L * U) pieces; workgroup w takes piece w % that of chunk
// w / that, and a piece past the end of its segment's last chunk does
// nothing.  The grid is two-dimensional (w = blockIdx.y * gridDim.x +
// blockIdx.x) because one dimension holds fewer than 2^32 lanes; workgroups
// past the last piece exit at once.  The segment depends on the chunk alone,
// so finding it runs on the scalar unit, once per wave: one load from the
// plan's chunk table (chunk_seg, by default), or a binary search whose upper
// levels stay in the scalar cache for every workgroup in flight.  With the
// search, small pieces repeat it for little data (256 lanes of one unit ran
// about 20% slower than 64 lanes of four); with the table, 1 KB pieces are
// the fastest shape.
//
// xcd_share != 0: the first 8 * xcd_share workgroups are renumbered so that
// each XCD (the hardware deals workgroups out to the 8 XCDs round-robin, so
// workgroup w runs on XCD w % 8) works through one contiguous share of them,
// in order: workgroup w takes piece (w % 8) * xcd_share + w / 8.  The
// workgroups resident on one XCD then touch a window of the plan one eighth
// as wide as when all eight XCDs share one window, so that XCD's L2 and
// address-translation caches hold fewer pages at a time.  The rest (fewer
// than 8) keep their own numbers.
template <bool kNT, bool kTable, int L, int U, bool kBuf>
__global__ __launch_bounds__(L) void copy_plan_kernel(const DevSeg *__restrict__ segs, uint64_t n_chunks,
                                                      SegHint hint, Bases src, Bases dst,
                                                      const uint64_t *__restrict__ src_tab,
                                                      const uint64_t *__restrict__ dst_tab, uint64_t xcd_share,
                                                      const uint32_t *__restrict__ chunk_seg) {
  constexpr uint32_t kPieces = kChunkUnits / (L * U);  // pieces per chunk: 1, 2 or 4
  static_assert(kPieces * L * U == kChunkUnits, "a piece divides a chunk");
  uint64_t w = (uint64_t)blockIdx.y * gridDim.x + blockIdx.x;
  if (w < xcd_share * 8) w = (w & 7) * xcd_share + (w >> 3);
  const uint64_t c = w / kPieces;
  if (c >= n_chunks) return;
  uint32_t lo;
  if (chunk_seg) {  // the segment of every chunk, looked up
    lo = chunk_seg[c];
  } else {  // found by a binary search bounded by the hint
    const uint32_t b = (uint32_t)(c >> hint.shift);
    lo = hint.first[b];
    uint32_t hi = hint.first[b + 1];
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1) >> 1;
      if (segs[mid].chunk_begin <= c) lo = mid;
      else hi = mid - 1;
    }
  }
  const DevSeg s = segs[lo];
  const uint32_t total = s.len * s.rows;
  const uint32_t u0 = (uint32_t)(c - s.chunk_begin) * kChunkUnits + (uint32_t)(w % kPieces) * (L * U);
  if (kPieces > 1 && u0 >= total) return;
  const char *sb = base_of<kTable>(src, src_tab, s.src_buf());
  char *db = base_of<kTable>(dst, dst_tab, s.dst_buf());
  char *ab = base_of<kTable>(dst, dst_tab, s.aux_buf());
  const uint32_t ops = s.ops(), ul = s.unit_log2();
  if constexpr (kBuf) {  // every unit width through buffer instructions
    if (ops & 4) {
      if (ops & 2) dispatch_chunk_buf<kNT, true, true, L, U>(ul, s, sb, db, ab, u0, total);
      else dispatch_chunk_buf<kNT, false, true, L, U>(ul, s, sb, db, ab, u0, total);
    } else if (ops & 1) {  // with the bf16 image (fp32 only: 16- or 4-byte units)
      if (ops & 2) {
        if (ul == 4) copy_units_buf<u32x4, kNT, true, true, false, L, U>(s, sb, db, ab, u0, total);
        else copy_units_buf<uint32_t, kNT, true, true, false, L, U>(s, sb, db, ab, u0, total);
      } else {
        if (ul == 4) copy_units_buf<u32x4, kNT, true, false, false, L, U>(s, sb, db, ab, u0, total);
        else copy_units_buf<uint32_t, kNT, true, false, false, L, U>(s, sb, db, ab, u0, total);
      }
    } else if (ops & 2) {
      dispatch_chunk_buf<kNT, true, false, L, U>(ul, s, sb, db, ab, u0, total);
    } else {
      dispatch_chunk_buf<kNT, false, false, L, U>(ul, s, sb, db, ab, u0, total);
    }
    return;
  }
  if (ops & 4) {  // duplicate to aux, with or without zero fill
    if (ops & 2) dispatch_chunk<kNT, true, true, L, U>(ul, s, sb, db, ab, u0, total);
    else dispatch_chunk<kNT, false, true, L, U>(ul, s, sb, db, ab, u0, total);
  } else if (ops & 1) {  // with the bf16 image (fp32 only: 16- or 4-byte units), with or without zero fill
    if (ops & 2) {
      if (ul == 4) copy_units<u32x4, kNT, true, true, false, L, U>(s, sb, db, ab, u0, total);
      else copy_units<uint32_t, kNT, true, true, false, L, U>(s, sb, db, ab, u0, total);
    } else {
      if (ul == 4) copy_units<u32x4, kNT, true, false, false, L, U>(s, sb, db, ab, u0, total);
      else copy_units<uint32_t, kNT, true, false, false, L, U>(s, sb, db, ab, u0, total);
    }
  } else if (ops & 2) {
    dispatch_chunk<kNT, true, false, L, U>(ul, s, sb, db, ab, u0, total);
  } else {
    dispatch_chunk<kNT, false, false, L, U>(ul, s, sb, db, ab, u0, total);
  }
}

// Reads a plan's lookup tables (its chunk table, then its segment
// descriptors) once, with cached loads, just before the copy.  Every copy
// workgroup starts with a dependent load from the chunk table: after
// unrelated work those loads miss every cache, each workgroup waits on HBM
// before its first data load, and the launch ran 4.5% slower than one
// straight after another copy (whose table reads left the table in the
// memory-side cache).  Read here first, at HBM speed and with every load in
// flight at once, the tables are in that cache when the copy starts.  The
// XOR only keeps the loads; nothing is stored.
__global__ __launch_bounds__(256) void warm_tables_kernel(const u32x4 *__restrict__ a, uint64_t na,
                                                          const u32x4 *__restrict__ b, uint64_t nb) {
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  uint32_t acc = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < na + nb; i += stride) {
    const u32x4 v = i < na ? a[i] : b[i - na];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  asm volatile("" ::"v"(acc));
}

// Writes the chunk table from the device segment table: segment k owns the
// chunks from its chunk_begin to the next segment's.  Built here, on the
// device, a plan's first call costs a few microseconds instead of a host fill
// and an upload of 4 bytes per chunk (79 MB on Llama-2-7B, about 27 ms).
__global__ __launch_bounds__(256) void fill_chunk_table_kernel(const DevSeg *__restrict__ segs, uint32_t nseg,
                                                               uint64_t n_chunks, uint32_t *__restrict__ out) {
  for (uint32_t k = blockIdx.x; k < nseg; k += gridDim.x) {
    const uint64_t c0 = segs[k].chunk_begin;
    const uint64_t c1 = k + 1 < nseg ? segs[k + 1].chunk_begin : n_chunks;
    for (uint64_t c = c0 + threadIdx.x; c < c1; c += 256) out[c] = k;
  }
}

// ---------------------------------------------------------------------------
// Device bookkeeping
// ---------------------------------------------------------------------------

struct DeviceProps {
  int cus = 0;
  int resident_blocks[2] = {0, 0};  // copy_plan_persistent_kernel<false/true> blocks per CU
};

std::mutex g_dev_mu;
std::vector<DeviceProps> g_dev_props;

template <bool kNT>
void persistent_occupancy(int *out) {
  int v = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, copy_plan_persistent_kernel<kNT, false>, kThreads, 0) !=
          hipSuccess ||
      v <= 0) {
    (void)hipGetLastError();
    v = 4;
  }
  *out = v;
}

int current_device(int *dev, int *cus, int *resident_nt, int *resident_t) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    (void)hipGetLastError();
    return fail(EMRS_ERR_NO_DEVICE, "no HIP device is visible");
  }
  e = hipGetDevice(dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_dev_mu);
  if ((int)g_dev_props.size() < n) g_dev_props.resize(n);
  if (g_dev_props[*dev].cus == 0) {
    int v = 0;
    e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, *dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
    g_dev_props[*dev].cus = v > 0 ? v : 1;
    persistent_occupancy<false>(&g_dev_props[*dev].resident_blocks[0]);
    persistent_occupancy<true>(&g_dev_props[*dev].resident_blocks[1]);
  }
  *cus = g_dev_props[*dev].cus;
  *resident_t = g_dev_props[*dev].resident_blocks[0];
  *resident_nt = g_dev_props[*dev].resident_blocks[1];
  return EMRS_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Plan
// ---------------------------------------------------------------------------

struct emrs_plan {
  std::vector<DevSeg> segs;
  std::vector<uint32_t> origin;              // input segment of each device segment
  uint64_t n_chunks = 0;
  SegHint hint{};                            // search bounds of the one-workgroup-per-chunk kernel
  std::vector<uint64_t> src_bytes, dst_bytes;
  std::vector<uint8_t> src_used, dst_used;  // buffers referenced by a non-empty segment
  emrs_plan_stats stats{};
  std::mutex mu;
  std::vector<DevSeg *> dev_tables;  // per device, uploaded on first use
  // Per device, uploaded on first use when emrs_tuning.chunk_index is set:
  // the device segment of every chunk (4 bytes per 4 KB chunk).
  std::vector<uint32_t *> chunk_tables;
  // Plans with more than kArgBuffers buffers on a side: per device, the
  // pointer table of the first execution and the base pointers it holds.
  std::vector<uint64_t *> ptr_tables;
  std::vector<std::vector<uint64_t>> ptr_contents;
  // For those same bases: the segment table with every offset made absolute
  // (units from abs_base, the lowest referenced base), per device.
  std::vector<DevSeg *> abs_tables;
  std::vector<uint64_t> abs_base;
  // Per device: one event recorded after each launch that may still be running (an event is
  // reused once its launch has finished).  Destroying the plan frees its tables in stream order
  // after these launches, and waits for nothing else.
  std::vector<std::vector<hipEvent_t>> launch_events;
  bool captured = false;  // a launch was recorded into a graph: destroy drains the device first
};

namespace {

// The plan's own device tables are stream-ordered allocations: made and
// filled synchronously on first use, and freed by emrs_plan_destroy on a
// library stream once the plan's launches have finished.
hipError_t table_alloc(void **out, size_t bytes, hipStream_t st) {
  *out = nullptr;
  const hipError_t e = hipMallocAsync(out, bytes, st);
  if (e != hipSuccess) *out = nullptr;
  return e;
}

int table_upload(void **out, const void *host, size_t bytes, hipStream_t st, const char *what) {
  hipError_t e = table_alloc(out, bytes, st);
  if (e != hipSuccess) return hip_fail(e, what);
  e = hipMemcpyAsync(*out, host, bytes, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);  // complete before any stream may read it
  if (e != hipSuccess) {
    (void)hipFreeAsync(*out, st);
    (void)hipStreamSynchronize(st);
    *out = nullptr;
    return hip_fail(e, what);
  }
  return EMRS_OK;
}

// Per device, the library's own stream on which destroyed plans free their
// tables (default priority, not blocking the null stream); nullptr if it
// could not be made.
hipStream_t free_stream(int dev) {
  static std::mutex mu;
  static std::vector<hipStream_t> streams;
  std::lock_guard<std::mutex> lk(mu);
  if ((int)streams.size() <= dev) streams.resize(dev + 1, nullptr);
  if (!streams[dev]) {
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess) streams[dev] = s;
    else (void)hipGetLastError();
  }
  return streams[dev];
}

// Record that the plan's tables are in use by the work just enqueued on `st`.
// Under graph capture nothing is recorded: the graph may replay any time, so
// destroy then drains the device instead.
int note_launch(emrs_plan *plan, int dev, hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  std::lock_guard<std::mutex> lk(plan->mu);
  if (cs != hipStreamCaptureStatusNone) {
    plan->captured = true;
    return EMRS_OK;
  }
  if ((int)plan->launch_events.size() <= dev) plan->launch_events.resize(dev + 1);
  std::vector<hipEvent_t> &evs = plan->launch_events[dev];
  hipEvent_t ev = nullptr;
  bool not_ready = false;
  for (hipEvent_t x : evs) {
    const hipError_t q = hipEventQuery(x);
    if (q == hipSuccess) {  // its launch has finished: reuse it
      ev = x;
      break;
    }
    not_ready = not_ready || q == hipErrorNotReady;
  }
  // A running launch's query answers hipErrorNotReady, which is no failure: do not leave it
  // behind as this thread's last error.
  if (not_ready) (void)hipGetLastError();
  if (!ev) {
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags");
    evs.push_back(ev);
  }
  e = hipEventRecord(ev, st);
  if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
  return EMRS_OK;
}

// Second destination of a segment: its bf16 image (cast; offsets in units
// of half the segment's unit) or a duplicate (dup; offsets in the segment's
// own units): buffer, offset and row stride.
struct Aux {
  bool on = false;    // cast or dup
  bool cast = false;  // EMRS_SEG_CAST_BF16
  bool dup = false;   // EMRS_SEG_DUP
  bool zero = false;  // the segment writes zeros (EMRS_SEG_ZERO_FILL)
  uint32_t buf = 0;
  uint64_t off = 0, stride = 0;
};

struct Builder {
  std::vector<DevSeg> out;
  std::vector<uint32_t> origin;  // input segment of each pushed segment
  uint32_t cur_origin = 0;       // input segment being emitted
  uint8_t cur_elem_log2 = 0;     // its element size
  uint64_t chunks = 0;
  uint64_t vec_bytes = 0, scalar_bytes = 0;

  // A copy in units of (1 << ul) bytes, optionally with its bf16 image.
  // Splits to the kernel's 32-bit limits.
  void emit(uint32_t sbuf, uint32_t dbuf, uint32_t ul, uint64_t so, uint64_t dof, uint64_t len,
            uint64_t rows, uint64_t ss, uint64_t ds, Aux ax = Aux()) {
    if (len == 0 || rows == 0) return;
    if (rows > 1 && ss == len && ds == len && (!ax.on || ax.stride == len)) {  // contiguous
      len *= rows;
      rows = 1;
    }
    (ul == 4 ? vec_bytes : scalar_bytes) += (len * rows) << ul;
    if (rows == 1) {
      for (uint64_t off = 0; off < len; off += kMaxUnitsPerSeg) {
        const uint64_t n = std::min<uint64_t>(kMaxUnitsPerSeg, len - off);
        push(sbuf, dbuf, ul, so + off, dof + off, (uint32_t)n, 1, 0, 0, ax, ax.off + off, 0);
      }
      return;
    }
    // Bytes per second-destination unit: half a unit for a bf16 image, a whole one for a duplicate.
    const uint64_t aub = ax.on ? (ax.cast ? (1ull << ul) / 2 : (1ull << ul)) : 0;
    if (len >= kMaxUnitsPerSeg || (ss << ul) >= kMaxPitchBytes || (ds << ul) >= kMaxPitchBytes ||
        ax.stride * aub >= kMaxPitchBytes) {
      for (uint64_t r = 0; r < rows; ++r)
        for (uint64_t off = 0; off < len; off += kMaxUnitsPerSeg) {
          const uint64_t n = std::min<uint64_t>(kMaxUnitsPerSeg, len - off);
          push(sbuf, dbuf, ul, so + r * ss + off, dof + r * ds + off, (uint32_t)n, 1, 0, 0, ax,
               ax.off + r * ax.stride + off, 0);
        }
      return;
    }
    const uint64_t rows_per = std::max<uint64_t>(1, kMaxUnitsPerSeg / len);
    for (uint64_t r = 0; r < rows; r += rows_per) {
      const uint64_t n = std::min<uint64_t>(rows_per, rows - r);
      push(sbuf, dbuf, ul, so + r * ss, dof + r * ds, (uint32_t)len, (uint32_t)n, (uint32_t)ss, (uint32_t)ds,
           ax, ax.off + r * ax.stride, (uint32_t)ax.stride);
    }
  }

  void push(uint32_t sbuf, uint32_t dbuf, uint32_t ul, uint64_t so, uint64_t dof, uint32_t len, uint32_t rows,
            uint32_t ss, uint32_t ds, const Aux &ax, uint64_t aoff, uint32_t astride) {
    DevSeg d{};
    d.src_off = so;
    d.dst_off = dof;
    d.chunk_begin = chunks;
    d.len = len;
    d.rows = rows;
    d.src_stride = rows > 1 ? ss : 0;
    d.dst_stride = rows > 1 ? ds : 0;
    uint32_t sh1 = 0, sh2 = 0;
    make_magic(len, &d.magic, &sh1, &sh2);
    const uint32_t ops = (ax.cast ? 1u : 0u) | (ax.zero ? 2u : 0u) | (ax.dup ? 4u : 0u);
    d.set_kind(sh2, sh1, ul, cur_elem_log2, ops);
    d.set_bufs(sbuf, dbuf, ax.on ? ax.buf : dbuf);
    d.aux_off = ax.on ? aoff : 0;
    d.aux_stride = ax.on && rows > 1 ? astride : 0;
    const uint64_t units = (uint64_t)len * rows;
    chunks += (units + kChunkUnits - 1) / kChunkUnits;
    out.push_back(d);
    origin.push_back(cur_origin);
  }
};

// Search bounds per bucket of 2^shift chunks, with at most kHintBuckets
// buckets: first[b] is the segment holding chunk b << shift (the last segment
// past the end).
void make_hint(const std::vector<DevSeg> &segs, uint64_t n_chunks, SegHint *h) {
  const uint32_t last = segs.empty() ? 0 : (uint32_t)segs.size() - 1;
  h->shift = 0;
  while (n_chunks && ((n_chunks - 1) >> h->shift) >= kHintBuckets) ++h->shift;
  for (uint32_t b = 0; b <= kHintBuckets; ++b) {
    const uint64_t c = (uint64_t)b << h->shift;
    if (c >= n_chunks) {
      h->first[b] = last;
      continue;
    }
    // Last segment whose first chunk is <= c.
    auto it = std::upper_bound(segs.begin(), segs.end(), c,
                               [](uint64_t v, const DevSeg &d) { return v < d.chunk_begin; });
    h->first[b] = (uint32_t)(it - segs.begin()) - 1;
  }
}

int log2_of(uint32_t eb) {
  switch (eb) {
    case 1: return 0;
    case 2: return 1;
    case 4: return 2;
    case 8: return 3;
    default: return -1;
  }
}

// Byte extent end of a strided segment (128-bit: cannot overflow).
unsigned __int128 extent_end(uint64_t off, uint64_t len, uint64_t rows, uint64_t stride, uint32_t eb) {
  return ((unsigned __int128)off + (unsigned __int128)(rows - 1) * stride + len) * eb;
}

int check_disjoint(const emrs_segment *segs, uint64_t n_segs) {
  struct Iv {
    uint32_t buf;
    uint64_t b, e;
  };
  uint64_t total_rows = 0;
  for (uint64_t i = 0; i < n_segs; ++i)
    if (segs[i].len) total_rows += segs[i].rows * ((segs[i].flags & (EMRS_SEG_CAST_BF16 | EMRS_SEG_DUP)) ? 2 : 1);
  if (total_rows > (1ull << 27))
    return fail(EMRS_ERR_INVALID_ARGUMENT, "disjointness check: too many rows to check");
  std::vector<Iv> iv;
  iv.reserve(total_rows);
  for (uint64_t i = 0; i < n_segs; ++i) {
    const emrs_segment &s = segs[i];
    if (!s.len) continue;
    for (uint64_t r = 0; r < s.rows; ++r) {
      const uint64_t b = (s.dst_off + r * s.dst_stride) * s.elem_bytes;
      iv.push_back({s.dst_buf, b, b + s.len * s.elem_bytes});
      if (s.flags & (EMRS_SEG_CAST_BF16 | EMRS_SEG_DUP)) {
        const uint64_t w = (s.flags & EMRS_SEG_CAST_BF16) ? 2 : s.elem_bytes;
        const uint64_t a = (s.aux_off + r * s.aux_stride) * w;
        iv.push_back({s.aux_buf, a, a + s.len * w});
      }
    }
  }
  std::sort(iv.begin(), iv.end(), [](const Iv &a, const Iv &b) { return a.buf != b.buf ? a.buf < b.buf : a.b < b.b; });
  for (size_t i = 1; i < iv.size(); ++i) {
    if (iv[i].buf == iv[i - 1].buf && iv[i].b < iv[i - 1].e) {
      char msg[160];
      snprintf(msg, sizeof msg, "destination ranges overlap in buffer %u at byte %llu", iv[i].buf,
               (unsigned long long)iv[i].b);
      return fail(EMRS_ERR_OVERLAP, msg);
    }
  }
  return EMRS_OK;
}

// Base pointers of an execution or comparison, checked (only buffers that
// some segment references) and laid out for the launch.
struct ResolvedBases {
  Bases src{}, dst{};
  bool table = false;         // pointers go through a device table: src then dst
  std::vector<uint64_t> ptrs;
};

// out_of_place: a destination buffer may overlap no other referenced buffer
// (an execution); a comparison only reads, so there any buffers may overlap.
int resolve_bases(const emrs_plan *plan, void *const *src_bases, void *const *dst_bases, ResolvedBases *rb,
                  bool out_of_place = true) {
  const uint32_t ns = plan->stats.n_src_bufs, nd = plan->stats.n_dst_bufs;
  if ((ns && !src_bases) || (nd && !dst_bases))
    return fail(EMRS_ERR_INVALID_ARGUMENT, "base pointer array is NULL");
  // Only buffers that some segment references are checked: an unreferenced
  // buffer may be NULL or alias anything.
  struct Iv {
    uintptr_t b, e;
    bool dst;
  };
  std::vector<Iv> iv;
  iv.reserve(ns + nd);
  for (uint32_t i = 0; i < ns; ++i) {
    if (!plan->src_used[i]) continue;
    const uintptr_t b = reinterpret_cast<uintptr_t>(src_bases[i]);
    if (!b) return fail(EMRS_ERR_INVALID_ARGUMENT, "source base is NULL");
    if (b % 16) return fail(EMRS_ERR_MISALIGNED, "source base is not 16-byte aligned");
    if (plan->src_bytes[i]) iv.push_back({b, b + plan->src_bytes[i], false});
  }
  for (uint32_t i = 0; i < nd; ++i) {
    if (!plan->dst_used[i]) continue;
    const uintptr_t b = reinterpret_cast<uintptr_t>(dst_bases[i]);
    if (!b) return fail(EMRS_ERR_INVALID_ARGUMENT, "destination base is NULL");
    if (b % 16) return fail(EMRS_ERR_MISALIGNED, "destination base is not 16-byte aligned");
    if (plan->dst_bytes[i]) iv.push_back({b, b + plan->dst_bytes[i], true});
  }
  // Out of place: no destination range may overlap another referenced range.
  // Sweep in address order; an earlier range overlaps the current one exactly
  // when its end lies past the current start.
  if (out_of_place) {
    std::sort(iv.begin(), iv.end(), [](const Iv &x, const Iv &y) { return x.b < y.b; });
    uintptr_t end_src = 0, end_dst = 0;
    for (const Iv &x : iv) {
      if (x.b < end_dst)
        return fail(EMRS_ERR_ALIAS, x.dst ? "two destination buffers overlap" : "a source buffer overlaps a destination buffer");
      if (x.dst && x.b < end_src) return fail(EMRS_ERR_ALIAS, "a source buffer overlaps a destination buffer");
      (x.dst ? end_dst : end_src) = std::max(x.dst ? end_dst : end_src, x.e);
    }
  }
  rb->table = ns > kArgBuffers || nd > kArgBuffers;
  if (rb->table) {
    rb->ptrs.resize((size_t)ns + nd);
    for (uint32_t i = 0; i < ns; ++i) rb->ptrs[i] = reinterpret_cast<uint64_t>(src_bases[i]);
    for (uint32_t i = 0; i < nd; ++i) rb->ptrs[ns + i] = reinterpret_cast<uint64_t>(dst_bases[i]);
  } else {
    for (uint32_t i = 0; i < ns; ++i) rb->src.p[i] = static_cast<char *>(src_bases[i]);
    for (uint32_t i = 0; i < nd; ++i) rb->dst.p[i] = static_cast<char *>(dst_bases[i]);
  }
  return EMRS_OK;
}

// The device pointer table of an execution or comparison (nullptr when the
// bases travel in kernel arguments).  The plan keeps, per device, the table of
// the first call and reuses it while the bases are the same: it is uploaded
// synchronously and never written again, so any stream may read it.  Calls
// with other bases get a stream-ordered table of their own (*owned = true),
// which the caller frees on the same stream after the launch.
int pointer_table(emrs_plan *plan, int dev, const ResolvedBases &rb, hipStream_t st, uint64_t **out, bool *owned) {
  *out = nullptr;
  *owned = false;
  if (!rb.table) return EMRS_OK;
  const size_t bytes = rb.ptrs.size() * sizeof(uint64_t);
  {
    std::lock_guard<std::mutex> lk(plan->mu);
    if ((int)plan->ptr_tables.size() <= dev) {
      plan->ptr_tables.resize(dev + 1, nullptr);
      plan->ptr_contents.resize(dev + 1);
    }
    if (plan->ptr_tables[dev]) {
      if (plan->ptr_contents[dev] == rb.ptrs) {
        *out = plan->ptr_tables[dev];
        return EMRS_OK;
      }
    } else {
      if (int rc = refuse_capture(st, "the first call of a plan on a device")) return rc;
      uint64_t *t = nullptr;
      if (int rc = table_upload(reinterpret_cast<void **>(&t), rb.ptrs.data(), bytes, st, "uploading the pointer table"))
        return rc;
      plan->ptr_tables[dev] = t;
      plan->ptr_contents[dev] = rb.ptrs;
      *out = t;
      return EMRS_OK;
    }
  }
  // Other bases than the cached ones: a table of this call's own, which a
  // captured graph could not replay (its host copy is this call's).
  if (int rc = refuse_capture(st, "a call whose base pointers differ from the plan's first call")) return rc;
  *owned = true;
  hipError_t e = hipMallocAsync(reinterpret_cast<void **>(out), bytes, st);
  if (e != hipSuccess) {
    *out = nullptr;
    return hip_fail(e, "hipMallocAsync(pointer table)");
  }
  e = hipMemcpyAsync(*out, rb.ptrs.data(), bytes, hipMemcpyHostToDevice, st);
  if (e != hipSuccess) {
    (void)hipFreeAsync(*out, st);
    *out = nullptr;
    return hip_fail(e, "hipMemcpyAsync(pointer table)");
  }
  return EMRS_OK;
}

// The plan's segment table on device `dev` resolved against the bases of its
// cached pointer table: every offset counts units from *common, the lowest
// referenced base, and every buffer id is 0, so the copy kernel looks up no
// base pointer at all.  Built and uploaded synchronously on first use, like
// the pointer table, and never written again.  *out = nullptr when the bases
// are not the cached ones (the caller then uses the pointer table).
int resolved_table(emrs_plan *plan, int dev, const ResolvedBases &rb, hipStream_t st, DevSeg **out,
                   char **common) {
  *out = nullptr;
  std::lock_guard<std::mutex> lk(plan->mu);
  if ((int)plan->ptr_tables.size() <= dev || !plan->ptr_tables[dev] || plan->ptr_contents[dev] != rb.ptrs)
    return EMRS_OK;
  if ((int)plan->abs_tables.size() <= dev) {
    plan->abs_tables.resize(dev + 1, nullptr);
    plan->abs_base.resize(dev + 1, 0);
  }
  if (!plan->abs_tables[dev]) {
    if (int rc = refuse_capture(st, "the first call of a plan on a device")) return rc;
    const uint32_t ns = plan->stats.n_src_bufs, nd = plan->stats.n_dst_bufs;
    uint64_t lo = ~0ull;
    for (uint32_t i = 0; i < ns; ++i)
      if (plan->src_used[i]) lo = std::min(lo, rb.ptrs[i]);
    for (uint32_t i = 0; i < nd; ++i)
      if (plan->dst_used[i]) lo = std::min(lo, rb.ptrs[ns + i]);
    // Referenced bases are 16-byte aligned, so every difference is a whole
    // number of units.  Unreferenced buffers (a zero fill's source) may be
    // NULL; their offsets are never used.
    auto units_from_lo = [lo](uint64_t p, uint32_t log2) -> uint64_t { return p >= lo ? (p - lo) >> log2 : 0; };
    std::vector<DevSeg> segs = plan->segs;
    for (DevSeg &d : segs) {
      const uint32_t ul = d.unit_log2(), ops = d.ops();
      const uint32_t aux_log2 = (ops & 1) ? ul - 1 : ul;  // a bf16 image unit is half a unit
      d.src_off = (ops & 2) ? 0 : d.src_off + units_from_lo(rb.ptrs[d.src_buf()], ul);
      d.dst_off += units_from_lo(rb.ptrs[ns + d.dst_buf()], ul);
      d.aux_off += units_from_lo(rb.ptrs[ns + d.aux_buf()], aux_log2);
      d.set_bufs(0, 0, 0);
    }
    const size_t bytes = segs.size() * sizeof(DevSeg);
    DevSeg *t = nullptr;
    if (int rc = table_upload(reinterpret_cast<void **>(&t), segs.data(), bytes, st, "uploading the resolved plan table"))
      return rc;
    plan->abs_tables[dev] = t;
    plan->abs_base[dev] = lo;
  }
  *out = plan->abs_tables[dev];
  *common = reinterpret_cast<char *>(plan->abs_base[dev]);
  return EMRS_OK;
}

// The device segment of every chunk on device `dev`, written on the device
// from its segment table `segs` on first use and never written again.
int chunk_table(emrs_plan *plan, int dev, hipStream_t st, const DevSeg *segs, uint32_t **out) {
  std::lock_guard<std::mutex> lk(plan->mu);
  if ((int)plan->chunk_tables.size() <= dev) plan->chunk_tables.resize(dev + 1, nullptr);
  if (!plan->chunk_tables[dev]) {
    // The table only spares each workgroup its search.  While the stream captures a graph it
    // cannot be built (that would record an allocation), so the launch searches instead; a
    // later call outside a capture builds it.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t ce = hipStreamIsCapturing(st, &cs);
    if (ce != hipSuccess) return hip_fail(ce, "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone) {
      *out = nullptr;
      return EMRS_OK;
    }
    if (plan->segs.size() > 0xffffffffull) return fail(EMRS_ERR_INVALID_ARGUMENT, "too many device segments");
    const size_t bytes = plan->n_chunks * sizeof(uint32_t);
    uint32_t *t = nullptr;
    hipError_t e = table_alloc(reinterpret_cast<void **>(&t), bytes, st);
    if (e == hipErrorOutOfMemory) {
      // The table only spares each workgroup its search: with no room for it,
      // this launch searches instead, and the next call tries again.
      (void)hipGetLastError();
      *out = nullptr;
      return EMRS_OK;
    }
    if (e != hipSuccess) return hip_fail(e, "hipMallocAsync(chunk table)");
    const uint32_t nseg = (uint32_t)plan->segs.size();
    hipLaunchKernelGGL(fill_chunk_table_kernel, dim3(std::min<uint32_t>(nseg, 65535)), dim3(256), 0, st, segs, nseg,
                       plan->n_chunks, t);
    e = hipGetLastError();
    // Later calls may come on other streams: the table is complete before it is published.
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
      (void)hipFreeAsync(t, st);
      (void)hipStreamSynchronize(st);
      return hip_fail(e, "building the chunk table");
    }
    plan->chunk_tables[dev] = t;
  }
  *out = plan->chunk_tables[dev];
  return EMRS_OK;
}

// The chunk table already on device `dev`, or nullptr: allocates nothing.
const uint32_t *existing_chunk_table(emrs_plan *plan, int dev) {
  std::lock_guard<std::mutex> lk(plan->mu);
  return (int)plan->chunk_tables.size() > dev ? plan->chunk_tables[dev] : nullptr;
}

// The plan's segment table on device `dev`, uploaded on first use.
int device_table(emrs_plan *plan, int dev, hipStream_t st, DevSeg **table) {
  std::lock_guard<std::mutex> lk(plan->mu);
  if ((int)plan->dev_tables.size() <= dev) plan->dev_tables.resize(dev + 1, nullptr);
  if (!plan->dev_tables[dev]) {
    if (int rc = refuse_capture(st, "the first call of a plan on a device")) return rc;
    const size_t bytes = plan->segs.size() * sizeof(DevSeg);
    DevSeg *t = nullptr;
    if (int rc = table_upload(reinterpret_cast<void **>(&t), plan->segs.data(), bytes, st, "uploading the plan table"))
      return rc;
    plan->dev_tables[dev] = t;
  }
  *table = plan->dev_tables[dev];
  return EMRS_OK;
}

// ---------------------------------------------------------------------------
// Compare kernel
// ---------------------------------------------------------------------------

// Device accumulators of one group (emrs_compare_stats minus the element
// count, which the host knows).  Maxima are non-negative floats, ordered as
// their bit patterns.
struct GroupAcc {
  unsigned long long mismatches;
  unsigned long long nonfinite;
  double sum_sq_diff;
  double sum_sq_expected;
  unsigned int max_abs_bits;
  unsigned int max_rel_bits;
};

struct LaneAcc {
  uint32_t mismatches = 0, nonfinite = 0;
  double sq_diff = 0.0, sq_exp = 0.0;
  float max_abs = 0.0f, max_rel = 0.0f;
};

__device__ __forceinline__ void cmp_float(LaneAcc &a, uint32_t e_bits, uint32_t g_bits) {
  const float e = __uint_as_float(e_bits), g = __uint_as_float(g_bits);
  if (fabsf(e) <= 3.402823466e38f) a.sq_exp += (double)e * (double)e;
  if (e_bits == g_bits) return;
  ++a.mismatches;
  const float d = fabsf(g - e);
  if (!(d <= 3.402823466e38f)) {  // NaN or infinite difference
    ++a.nonfinite;
    return;
  }
  a.sq_diff += (double)d * (double)d;
  a.max_abs = fmaxf(a.max_abs, d);
  a.max_rel = fmaxf(a.max_rel, d / (fabsf(e) + 1e-12f));
}

// Compare one unit (1, 2, 4, 8 or 16 bytes held in w[0..3]) element by element.
__device__ __forceinline__ void cmp_words(LaneAcc &a, const uint32_t *e, const uint32_t *g, uint32_t unit_bytes,
                                          uint32_t elem_log2) {
  switch (elem_log2) {
    case 2:  // fp32
      for (uint32_t k = 0; k < unit_bytes / 4; ++k) cmp_float(a, e[k], g[k]);
      break;
    case 1:  // bf16
      for (uint32_t k = 0; k < unit_bytes / 2; ++k) {
        const uint32_t sh = (k & 1) * 16;
        cmp_float(a, ((e[k >> 1] >> sh) & 0xffffu) << 16, ((g[k >> 1] >> sh) & 0xffffu) << 16);
      }
      break;
    case 0:  // bytes: bits only
      for (uint32_t k = 0; k < unit_bytes; ++k) {
        const uint32_t sh = (k & 3) * 8;
        a.mismatches += ((e[k >> 2] >> sh) & 0xffu) != ((g[k >> 2] >> sh) & 0xffu);
      }
      break;
    default:  // 8-byte elements: bits only
      for (uint32_t k = 0; k < unit_bytes / 8; ++k)
        a.mismatches += (e[2 * k] != g[2 * k]) || (e[2 * k + 1] != g[2 * k + 1]);
      break;
  }
}

template <typename T>
__device__ __forceinline__ void words_of(const T &v, uint32_t *w) {
  if constexpr (sizeof(T) == 16) {
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (sizeof(T) == 8) {
    w[0] = (uint32_t)v; w[1] = (uint32_t)(v >> 32);
  } else {
    w[0] = (uint32_t)v;
  }
}

template <typename A>
__device__ __forceinline__ void aux_words_of(const A &v, uint32_t *w) {
  if constexpr (sizeof(A) == 8) {
    w[0] = v.x; w[1] = v.y;
  } else {
    w[0] = (uint32_t)v;
  }
}

// Compare units [u0, u_end) of segment s (at most kStepUnits); with a cast,
// also its bf16 image; with a duplicate, also the second copy.
template <typename T>
__device__ __forceinline__ void compare_chunk(const DevSeg &s, const char *sbase, const char *dbase,
                                              const char *abase, uint32_t u0, uint32_t u_end, LaneAcc &m,
                                              LaneAcc &x) {
  typedef typename std::conditional<sizeof(T) == 16 || sizeof(T) == 4, CastOf<T>, CastOf<uint32_t>>::type C;
  typedef typename C::type A;
  const T *src = reinterpret_cast<const T *>(sbase);
  const T *dst = reinterpret_cast<const T *>(dbase);
  const A *aux = reinterpret_cast<const A *>(abase);
  for (uint32_t j = 0; j < kUnroll; ++j) {
    const uint32_t u = u0 + j * kThreads + threadIdx.x;
    if (u >= u_end) break;
    uint64_t so = s.src_off + u, dof = s.dst_off + u, ao = s.aux_off + u;
    if (s.rows > 1) {
      const uint32_t row = magic_div(u, s.magic, s.sh1(), s.sh2()), col = u - row * s.len;
      so = s.src_off + (uint64_t)row * s.src_stride + col;
      dof = s.dst_off + (uint64_t)row * s.dst_stride + col;
      ao = s.aux_off + (uint64_t)row * s.aux_stride + col;
    }
    const uint32_t ops = s.ops();
    const T e = (ops & 2) ? T{} : ld<T, true>(src + so);
    const T g = ld<T, true>(dst + dof);
    uint32_t ew[4] = {0, 0, 0, 0}, gw[4] = {0, 0, 0, 0};
    words_of(e, ew);
    words_of(g, gw);
    cmp_words(m, ew, gw, (uint32_t)sizeof(T), s.elem_log2());
    if (ops & 4) {
      uint32_t dw[4] = {0, 0, 0, 0};
      words_of(ld<T, true>(reinterpret_cast<const T *>(abase) + ao), dw);
      cmp_words(x, ew, dw, (uint32_t)sizeof(T), s.elem_log2());
    }
    if constexpr (sizeof(T) == 16 || sizeof(T) == 4) {
      if (ops & 1) {
        uint32_t ea[2] = {0, 0}, ga[2] = {0, 0};
        aux_words_of(C::cast(e), ea);
        aux_words_of(ld<A, true>(aux + ao), ga);
        cmp_words(x, ea, ga, (uint32_t)sizeof(A), 1);
      }
    }
  }
}

// Bits of a that differ from b, folded into one word (0: the units are equal).
__device__ __forceinline__ uint32_t differ(const u32x4 &a, const u32x4 &b) {
  return (a.x ^ b.x) | (a.y ^ b.y) | (a.z ^ b.z) | (a.w ^ b.w);
}
__device__ __forceinline__ uint32_t differ(uint64_t a, uint64_t b) {
  const uint64_t d = a ^ b;
  return (uint32_t)d | (uint32_t)(d >> 32);
}
__device__ __forceinline__ uint32_t differ(uint32_t a, uint32_t b) { return a ^ b; }
__device__ __forceinline__ uint32_t differ(uint16_t a, uint16_t b) { return (uint32_t)(a ^ b); }
__device__ __forceinline__ uint32_t differ(uint8_t a, uint8_t b) { return (uint32_t)(a ^ b); }
__device__ __forceinline__ uint32_t differ(const CastOf<u32x4>::type &a, const CastOf<u32x4>::type &b) {
  return (a.x ^ b.x) | (a.y ^ b.y);
}

// The bit-level pass over units [u0, u_end) of segment s: `dm` collects the
// bits in which the destination differs from the source, `dx` those of the
// second destination (bf16 image or duplicate).  Loads, addresses and order
// are compare_chunk's; only the arithmetic is left out.
template <typename T>
__device__ __forceinline__ void differ_chunk(const DevSeg &s, const char *sbase, const char *dbase,
                                             const char *abase, uint32_t u0, uint32_t u_end, uint32_t &dm,
                                             uint32_t &dx) {
  typedef typename std::conditional<sizeof(T) == 16 || sizeof(T) == 4, CastOf<T>, CastOf<uint32_t>>::type C;
  typedef typename C::type A;
  const T *src = reinterpret_cast<const T *>(sbase);
  const T *dst = reinterpret_cast<const T *>(dbase);
  const A *aux = reinterpret_cast<const A *>(abase);
  const T *dup = reinterpret_cast<const T *>(abase);
  const uint32_t ops = s.ops();
  for (uint32_t j = 0; j < kUnroll; ++j) {
    const uint32_t u = u0 + j * kThreads + threadIdx.x;
    if (u >= u_end) break;
    uint64_t so = s.src_off + u, dof = s.dst_off + u, ao = s.aux_off + u;
    if (s.rows > 1) {
      const uint32_t row = magic_div(u, s.magic, s.sh1(), s.sh2()), col = u - row * s.len;
      so = s.src_off + (uint64_t)row * s.src_stride + col;
      dof = s.dst_off + (uint64_t)row * s.dst_stride + col;
      ao = s.aux_off + (uint64_t)row * s.aux_stride + col;
    }
    const T e = (ops & 2) ? T{} : ld<T, true>(src + so);
    dm |= differ(e, ld<T, true>(dst + dof));
    if (ops & 4) dx |= differ(e, ld<T, true>(dup + ao));
    if constexpr (sizeof(T) == 16 || sizeof(T) == 4) {
      if (ops & 1) dx |= differ(C::cast(e), ld<A, true>(aux + ao));
    }
  }
}

// First pass of a comparison on the copy kernel's schedule: one 64-lane
// workgroup per piece of U units of a chunk (U = 4: one workgroup per 4 KB
// chunk), its segment from the plan's chunk table, dispatched in order and,
// on large plans, each XCD on its own eighth of the pieces.  Every lane issues
// its U units' source and destination loads before it compares them.  Faster
// than the persistent grid on every full-size switch (2-4%, same allocations):
// a segment's rows or gathered runs are spread over many workgroups in flight.
template <typename T, int U>
__device__ __forceinline__ void differ_units(const DevSeg &s, const char *sbase, const char *dbase,
                                             const char *abase, uint32_t u0, uint32_t total, uint32_t &dm,
                                             uint32_t &dx) {
  typedef typename std::conditional<sizeof(T) == 16 || sizeof(T) == 4, CastOf<T>, CastOf<uint32_t>>::type C;
  typedef typename C::type A;
  const T *src = reinterpret_cast<const T *>(sbase);
  const T *dst = reinterpret_cast<const T *>(dbase);
  const A *aux = reinterpret_cast<const A *>(abase);
  const T *dup = reinterpret_cast<const T *>(abase);
  const uint32_t ops = s.ops();
  T e[U], g[U];
  uint64_t ao[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t u = u0 + j * 64 + threadIdx.x;
    e[j] = T{};
    g[j] = T{};
    ao[j] = 0;
    if (u < total) {
      uint64_t so = s.src_off + u, dof = s.dst_off + u;
      ao[j] = s.aux_off + u;
      if (s.rows > 1) {
        const uint32_t row = magic_div(u, s.magic, s.sh1(), s.sh2()), col = u - row * s.len;
        so = s.src_off + (uint64_t)row * s.src_stride + col;
        dof = s.dst_off + (uint64_t)row * s.dst_stride + col;
        ao[j] = s.aux_off + (uint64_t)row * s.aux_stride + col;
      }
      if (!(ops & 2)) e[j] = ld<T, true>(src + so);
      g[j] = ld<T, true>(dst + dof);
    }
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t u = u0 + j * 64 + threadIdx.x;
    if (u < total) {
      dm |= differ(e[j], g[j]);
      if (ops & 4) dx |= differ(e[j], ld<T, true>(dup + ao[j]));
      if constexpr (sizeof(T) == 16 || sizeof(T) == 4) {
        if (ops & 1) dx |= differ(C::cast(e[j]), ld<A, true>(aux + ao[j]));
      }
    }
  }
}

template <bool kTable, int U>
__global__ __launch_bounds__(64) void differ_piece_kernel(
    const DevSeg *__restrict__ segs, uint64_t n_chunks, Bases src, Bases dst, const uint64_t *__restrict__ src_tab,
    const uint64_t *__restrict__ dst_tab, uint64_t xcd_share, const uint32_t *__restrict__ chunk_seg,
    const uint32_t *__restrict__ groups, const uint32_t *__restrict__ aux_groups, GroupAcc *__restrict__ acc) {
  constexpr uint32_t kPieces = kChunkUnits / (64 * U);
  uint64_t w = (uint64_t)blockIdx.y * gridDim.x + blockIdx.x;
  if (w < xcd_share * 8) w = (w & 7) * xcd_share + (w >> 3);
  const uint64_t c = w / kPieces;
  if (c >= n_chunks) return;
  const uint32_t lo = chunk_seg[c];
  const DevSeg s = segs[lo];
  const uint32_t total = s.len * s.rows;
  const uint32_t u0 = (uint32_t)(c - s.chunk_begin) * kChunkUnits + (uint32_t)(w % kPieces) * (64 * U);
  if (kPieces > 1 && u0 >= total) return;
  const char *sb = base_of<kTable>(src, src_tab, s.src_buf());
  const char *db = base_of<kTable>(dst, dst_tab, s.dst_buf());
  const char *ab = base_of<kTable>(dst, dst_tab, s.aux_buf());
  uint32_t dm = 0, dx = 0;
  switch (s.unit_log2()) {
    case 4: differ_units<u32x4, U>(s, sb, db, ab, u0, total, dm, dx); break;
    case 3: differ_units<uint64_t, U>(s, sb, db, ab, u0, total, dm, dx); break;
    case 2: differ_units<uint32_t, U>(s, sb, db, ab, u0, total, dm, dx); break;
    case 1: differ_units<uint16_t, U>(s, sb, db, ab, u0, total, dm, dx); break;
    default: differ_units<uint8_t, U>(s, sb, db, ab, u0, total, dm, dx); break;
  }
  if (__any(dm != 0) && threadIdx.x == 0) atomicOr(&acc[groups[lo]].mismatches, 1ull);
  if ((s.ops() & 5) && __any(dx != 0) && threadIdx.x == 0) atomicOr(&acc[aux_groups[lo]].mismatches, 1ull);
}

// Mark the groups whose elements differ: one atomic per wave that saw a
// difference, none for a wave that saw none.  No barrier: each wave marks on
// its own.
__device__ __forceinline__ void mark_differ(uint32_t &dm, uint32_t &dx, uint32_t g, uint32_t ga, bool aux,
                                            GroupAcc *acc) {
  const bool lead = (threadIdx.x & 63) == 0;
  if (__any(dm != 0) && lead) atomicOr(&acc[g].mismatches, 1ull);
  if (aux && __any(dx != 0) && lead) atomicOr(&acc[ga].mismatches, 1ull);
  dm = dx = 0;
}

// First pass of a comparison when the plan has no chunk table on the device
// (it did not fit, or emrs_plan_compare_static meets a plan that has never
// run there): which groups differ at all, on compare_plan_kernel's persistent
// schedule.  Per lane only two words of differing bits are kept.  Only the
// groups it marks are compared again for compare_ckpt's figures
// (compare_plan_kernel), whose per-element fp64 work costs about 4% more time
// on Llama-2-7B than reading alone.
template <bool kTable>
__global__ __launch_bounds__(kThreads) void differ_plan_kernel(
    const DevSeg *__restrict__ segs, const uint32_t *__restrict__ groups, const uint32_t *__restrict__ aux_groups,
    uint32_t n_segs, uint64_t n_chunks, uint32_t run, Bases src, Bases dst, const uint64_t *__restrict__ src_tab,
    const uint64_t *__restrict__ dst_tab, GroupAcc *__restrict__ acc) {
  const uint64_t xcd = blockIdx.x & 7;
  const uint64_t c1 = n_chunks * (xcd + 1) / 8;
  const uint64_t step = (uint64_t)(gridDim.x >> 3) * run;
  uint32_t dm = 0, dx = 0, cur_g = 0, cur_ga = 0;
  bool open = false, cur_aux = false;
  for (uint64_t c = n_chunks * xcd / 8 + (uint64_t)(blockIdx.x >> 3) * run; c < c1; c += step) {
    const uint64_t c_end = min(c + run, c1);
    uint32_t lo = 0, hi = n_segs - 1;
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1) >> 1;
      if (segs[mid].chunk_begin <= c) lo = mid;
      else hi = mid - 1;
    }
    uint32_t si = lo;
    uint64_t s_end = (si + 1 < n_segs) ? segs[si + 1].chunk_begin : n_chunks;
    for (uint64_t q = c, nq; q < c_end; q += nq) {
      while (q >= s_end) {
        ++si;
        s_end = (si + 1 < n_segs) ? segs[si + 1].chunk_begin : n_chunks;
      }
      nq = min(min(c_end, s_end) - q, (uint64_t)kUnroll);
      const DevSeg s = segs[si];
      const uint32_t g = groups[si], ga = aux_groups[si];
      const bool aux = (s.ops() & 5) != 0;
      if (open && (g != cur_g || aux != cur_aux || (aux && ga != cur_ga))) mark_differ(dm, dx, cur_g, cur_ga, cur_aux, acc);
      open = true;
      cur_g = g;
      cur_ga = ga;
      cur_aux = aux;
      const uint32_t total = s.len * s.rows;
      const uint32_t u0 = (uint32_t)(q - s.chunk_begin) * kChunkUnits;
      const uint32_t u_end = min(u0 + (uint32_t)nq * kChunkUnits, total);
      const char *sb = base_of<kTable>(src, src_tab, s.src_buf());
      const char *db = base_of<kTable>(dst, dst_tab, s.dst_buf());
      const char *ab = base_of<kTable>(dst, dst_tab, s.aux_buf());
      switch (s.unit_log2()) {
        case 4: differ_chunk<u32x4>(s, sb, db, ab, u0, u_end, dm, dx); break;
        case 3: differ_chunk<uint64_t>(s, sb, db, ab, u0, u_end, dm, dx); break;
        case 2: differ_chunk<uint32_t>(s, sb, db, ab, u0, u_end, dm, dx); break;
        case 1: differ_chunk<uint16_t>(s, sb, db, ab, u0, u_end, dm, dx); break;
        default: differ_chunk<uint8_t>(s, sb, db, ab, u0, u_end, dm, dx); break;
      }
    }
  }
  if (open) mark_differ(dm, dx, cur_g, cur_ga, cur_aux, acc);
}

// Sum / max over the workgroup; the result is valid in thread 0.
__device__ void block_reduce(LaneAcc &a, double *lds_d, uint32_t *lds_u, float *lds_f) {
  for (int off = 32; off > 0; off >>= 1) {
    a.mismatches += __shfl_xor(a.mismatches, off, 64);
    a.nonfinite += __shfl_xor(a.nonfinite, off, 64);
    a.sq_diff += __shfl_xor(a.sq_diff, off, 64);
    a.sq_exp += __shfl_xor(a.sq_exp, off, 64);
    a.max_abs = fmaxf(a.max_abs, __shfl_xor(a.max_abs, off, 64));
    a.max_rel = fmaxf(a.max_rel, __shfl_xor(a.max_rel, off, 64));
  }
  const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  __syncthreads();
  if (lane == 0) {
    lds_u[2 * wave] = a.mismatches;
    lds_u[2 * wave + 1] = a.nonfinite;
    lds_d[2 * wave] = a.sq_diff;
    lds_d[2 * wave + 1] = a.sq_exp;
    lds_f[2 * wave] = a.max_abs;
    lds_f[2 * wave + 1] = a.max_rel;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (uint32_t w = 1; w < kThreads / 64; ++w) {
      a.mismatches += lds_u[2 * w];
      a.nonfinite += lds_u[2 * w + 1];
      a.sq_diff += lds_d[2 * w];
      a.sq_exp += lds_d[2 * w + 1];
      a.max_abs = fmaxf(a.max_abs, lds_f[2 * w]);
      a.max_rel = fmaxf(a.max_rel, lds_f[2 * w + 1]);
    }
  }
}

__device__ void flush(const LaneAcc &a, GroupAcc *g) {
  if (a.mismatches) atomicAdd(&g->mismatches, (unsigned long long)a.mismatches);
  if (a.nonfinite) atomicAdd(&g->nonfinite, (unsigned long long)a.nonfinite);
  if (a.sq_diff != 0.0) atomicAdd(&g->sum_sq_diff, a.sq_diff);
  if (a.sq_exp != 0.0) atomicAdd(&g->sum_sq_expected, a.sq_exp);
  if (a.max_abs > 0.0f) atomicMax(&g->max_abs_bits, __float_as_uint(a.max_abs));
  if (a.max_rel > 0.0f) atomicMax(&g->max_rel_bits, __float_as_uint(a.max_rel));
}

// Add the workgroup's lane sums to their groups and clear them: the values
// compared, and with `aux` the second destination's.  Every thread calls it.
__device__ void flush_block(LaneAcc &m, LaneAcc &x, uint32_t g, uint32_t ga, bool aux, GroupAcc *acc,
                            const uint8_t *active, double *lds_d, uint32_t *lds_u, float *lds_f) {
  if (active[g]) {
    block_reduce(m, lds_d, lds_u, lds_f);
    if (threadIdx.x == 0) flush(m, acc + g);
  }
  if (aux && active[ga]) {
    block_reduce(x, lds_d, lds_u, lds_f);
    if (threadIdx.x == 0) flush(x, acc + ga);
  }
  __syncthreads();  // the LDS slots are reused by the next reduction
  m = LaneAcc();
  x = LaneAcc();
}

// Workgroups take runs of `run` consecutive chunks, each XCD sweeping its own
// eighth of the plan (workgroup b runs on XCD b % 8; the grid is a multiple of
// 8), and compare up to kUnroll chunks of one segment per step, so that every
// lane has several loads in flight.  Lane sums stay in registers while consecutive
// chunks share their (group, aux group); they are reduced over the workgroup
// only when that pair changes and at the end.  Every decision depends on the
// segment alone, so it is uniform across the workgroup, and every thread
// reaches every barrier.  Only segments with a group marked in `active` are
// compared, and only marked groups are accumulated: the second pass of a
// comparison, over the groups the first pass (differ_plan_kernel) found to differ.
template <bool kTable>
__global__ __launch_bounds__(kThreads) void compare_plan_kernel(
    const DevSeg *__restrict__ segs, const uint32_t *__restrict__ groups, const uint32_t *__restrict__ aux_groups,
    uint32_t n_segs, uint64_t n_chunks, uint32_t run, Bases src, Bases dst, const uint64_t *__restrict__ src_tab,
    const uint64_t *__restrict__ dst_tab, GroupAcc *__restrict__ acc, const uint8_t *__restrict__ active) {
  __shared__ double lds_d[2 * kThreads / 64];
  __shared__ uint32_t lds_u[2 * kThreads / 64];
  __shared__ float lds_f[2 * kThreads / 64];
  const uint64_t xcd = blockIdx.x & 7;
  const uint64_t c1 = n_chunks * (xcd + 1) / 8;
  const uint64_t step = (uint64_t)(gridDim.x >> 3) * run;
  LaneAcc m, x;
  uint32_t cur_g = 0, cur_ga = 0;
  bool open = false, cur_aux = false;
  for (uint64_t c = n_chunks * xcd / 8 + (uint64_t)(blockIdx.x >> 3) * run; c < c1; c += step) {
    const uint64_t c_end = min(c + run, c1);
    uint32_t lo = 0, hi = n_segs - 1;
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1) >> 1;
      if (segs[mid].chunk_begin <= c) lo = mid;
      else hi = mid - 1;
    }
    uint32_t si = lo;
    uint64_t s_end = (si + 1 < n_segs) ? segs[si + 1].chunk_begin : n_chunks;
    for (uint64_t q = c, nq; q < c_end; q += nq) {
      while (q >= s_end) {
        ++si;
        s_end = (si + 1 < n_segs) ? segs[si + 1].chunk_begin : n_chunks;
      }
      nq = min(min(c_end, s_end) - q, (uint64_t)kUnroll);  // chunks of this segment in this step
      const DevSeg s = segs[si];
      const uint32_t g = groups[si], ga = aux_groups[si];
      const bool aux = (s.ops() & 5) != 0;  // cast or duplicate
      if (!active[g] && !(aux && active[ga])) continue;  // no group of this segment differs
      if (open && (g != cur_g || aux != cur_aux || (aux && ga != cur_ga)))
        flush_block(m, x, cur_g, cur_ga, cur_aux, acc, active, lds_d, lds_u, lds_f);
      open = true;
      cur_g = g;
      cur_ga = ga;
      cur_aux = aux;
      const uint32_t total = s.len * s.rows;
      const uint32_t u0 = (uint32_t)(q - s.chunk_begin) * kChunkUnits;
      const uint32_t u_end = min(u0 + (uint32_t)nq * kChunkUnits, total);
      const char *sb = base_of<kTable>(src, src_tab, s.src_buf());
      const char *db = base_of<kTable>(dst, dst_tab, s.dst_buf());
      const char *ab = base_of<kTable>(dst, dst_tab, s.aux_buf());
      switch (s.unit_log2()) {
        case 4: compare_chunk<u32x4>(s, sb, db, ab, u0, u_end, m, x); break;
        case 3: compare_chunk<uint64_t>(s, sb, db, ab, u0, u_end, m, x); break;
        case 2: compare_chunk<uint32_t>(s, sb, db, ab, u0, u_end, m, x); break;
        case 1: compare_chunk<uint16_t>(s, sb, db, ab, u0, u_end, m, x); break;
        default: compare_chunk<uint8_t>(s, sb, db, ab, u0, u_end, m, x); break;
      }
    }
  }
  if (open) flush_block(m, x, cur_g, cur_ga, cur_aux, acc, active, lds_d, lds_u, lds_f);
}

// Zero n 32-bit words (accumulators are cleared by a kernel rather than a memset).
__global__ void clear_words_kernel(uint32_t *p, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// What both comparison entry points prepare on the host: checked bases, the
// groups of every device segment, and the element counts per group.
struct CompareJob {
  ResolvedBases rb;
  std::vector<uint32_t> g_host;  // per device segment: its group, then its aux group
  int cus = 0;
  int resident = 0;              // compare_plan_kernel workgroups per CU
  int resident_differ = 0;       // differ_plan_kernel workgroups per CU
  const uint32_t *cseg = nullptr;  // the plan's chunk table on this device, if there is one
};

int compare_setup(emrs_plan *plan, void *const *src_bases, void *const *dst_bases, const uint32_t *groups,
                  const uint32_t *aux_groups, uint32_t n_groups, emrs_compare_stats *stats, CompareJob *job) {
  if (!plan || !stats) return fail(EMRS_ERR_INVALID_ARGUMENT, "NULL argument");
  if (n_groups == 0) return fail(EMRS_ERR_INVALID_ARGUMENT, "n_groups must be >= 1");
  const uint64_t n_in = plan->stats.n_segments;
  for (uint64_t i = 0; i < n_in; ++i)
    if ((groups && groups[i] >= n_groups) || (aux_groups && aux_groups[i] >= n_groups))
      return fail(EMRS_ERR_INVALID_ARGUMENT, "group id >= n_groups");
  int rc = resolve_bases(plan, src_bases, dst_bases, &job->rb, /*out_of_place=*/false);
  if (rc) return rc;
  const size_t nd = plan->segs.size();
  job->g_host.resize(2 * nd);
  std::vector<uint64_t> elements(n_groups, 0);
  for (size_t k = 0; k < nd; ++k) {
    const DevSeg &d = plan->segs[k];
    const uint32_t o = plan->origin[k];
    const uint32_t g = groups ? groups[o] : 0, ga = aux_groups ? aux_groups[o] : g;
    job->g_host[k] = g;
    job->g_host[nd + k] = ga;
    const uint64_t units = (uint64_t)d.len * d.rows;
    elements[g] += units << (d.unit_log2() - d.elem_log2());
    if (d.ops() & 1) elements[ga] += units << (d.unit_log2() - 2);
    if (d.ops() & 4) elements[ga] += units << (d.unit_log2() - d.elem_log2());
  }
  for (uint32_t g = 0; g < n_groups; ++g) {
    stats[g] = emrs_compare_stats{};
    stats[g].elements = elements[g];
  }
  return EMRS_OK;
}

// The current device, its CU count and the compare kernel's residency.
int compare_device(CompareJob *job, int *dev) {
  int resident_nt = 0, resident_t = 0;
  int rc = current_device(dev, &job->cus, &resident_nt, &resident_t);
  if (rc) return rc;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&job->resident, compare_plan_kernel<false>, kThreads, 0) !=
          hipSuccess ||
      job->resident <= 0) {
    (void)hipGetLastError();
    job->resident = 4;
  }
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&job->resident_differ, differ_plan_kernel<false>, kThreads, 0) !=
          hipSuccess ||
      job->resident_differ <= 0) {
    (void)hipGetLastError();
    job->resident_differ = job->resident;
  }
  return EMRS_OK;
}

// A persistent grid of resident workgroups, a multiple of 8 (one eighth of
// the plan per XCD), in runs of up to 32 steps: at most a quarter of each
// workgroup's share, so that small plans still spread out.  `active` null:
// the first pass (differ_piece_kernel with the plan's chunk table, else
// differ_plan_kernel); else the second (compare_plan_kernel).
hipError_t compare_launch(const emrs_plan *plan, const CompareJob &job, const DevSeg *table, const uint32_t *grp,
                          const uint64_t *tab, GroupAcc *acc, const uint8_t *active, hipStream_t st) {
  const size_t nd = plan->segs.size();
  // The first pass could hold 8 workgroups per CU; 3-6 read at the plain read rate and 8 is up to
  // 7% slower (Llama-2-7B, Mixtral and Group-ZeRO switches, same allocations): 4.
  const uint32_t resident = (uint32_t)(active ? job.resident : std::min(job.resident_differ, kDifferBlocksPerCu));
  uint64_t blocks = std::min<uint64_t>(plan->n_chunks, (uint64_t)job.cus * resident);
  blocks = std::max<uint64_t>(8, blocks / 8 * 8);
  const uint32_t run =
      (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(32 * kUnroll, plan->n_chunks / (blocks * 4)));
  const uint64_t *dtab = tab ? tab + plan->stats.n_src_bufs : nullptr;
  const dim3 grid((uint32_t)blocks), block(kThreads);
  if (!active && job.cseg) {  // the first pass on the copy kernel's schedule
    constexpr int U = 4;
    const uint64_t n_wg = plan->n_chunks * (kChunkUnits / (64 * U));
    const uint64_t gx = std::min<uint64_t>(n_wg, std::max<uint64_t>(1ull << 16, (n_wg + kMaxGridY - 1) / kMaxGridY));
    const dim3 pgrid((uint32_t)gx, (uint32_t)((n_wg + gx - 1) / gx));
    const uint32_t remap = g_tuning.xcd_remap.load();
    const bool by_xcd = remap == 2 || (remap == 1 && plan->n_chunks >= kXcdRemapMinChunks);
    const uint64_t xcd_share = by_xcd ? n_wg / 8 : 0;
    if (job.rb.table)
      hipLaunchKernelGGL((differ_piece_kernel<true, U>), pgrid, dim3(64), 0, st, table, plan->n_chunks, job.rb.src,
                         job.rb.dst, tab, dtab, xcd_share, job.cseg, grp, grp + nd, acc);
    else
      hipLaunchKernelGGL((differ_piece_kernel<false, U>), pgrid, dim3(64), 0, st, table, plan->n_chunks, job.rb.src,
                         job.rb.dst, tab, dtab, xcd_share, job.cseg, grp, grp + nd, acc);
    return hipGetLastError();
  }
  if (!active) {
    if (job.rb.table)
      hipLaunchKernelGGL(differ_plan_kernel<true>, grid, block, 0, st, table, grp, grp + nd, (uint32_t)nd,
                         plan->n_chunks, run, job.rb.src, job.rb.dst, tab, dtab, acc);
    else
      hipLaunchKernelGGL(differ_plan_kernel<false>, grid, block, 0, st, table, grp, grp + nd, (uint32_t)nd,
                         plan->n_chunks, run, job.rb.src, job.rb.dst, tab, dtab, acc);
  } else if (job.rb.table) {
    hipLaunchKernelGGL(compare_plan_kernel<true>, grid, block, 0, st, table, grp, grp + nd, (uint32_t)nd,
                       plan->n_chunks, run, job.rb.src, job.rb.dst, tab, dtab, acc, active);
  } else {
    hipLaunchKernelGGL(compare_plan_kernel<false>, grid, block, 0, st, table, grp, grp + nd, (uint32_t)nd,
                       plan->n_chunks, run, job.rb.src, job.rb.dst, tab, dtab, acc, active);
  }
  return hipGetLastError();
}

// Zero the accumulators with a kernel (no memset node if the stream's work is ever captured).
hipError_t clear_acc(GroupAcc *acc, uint32_t n_groups, hipStream_t st) {
  const uint64_t words = (uint64_t)n_groups * sizeof(GroupAcc) / sizeof(uint32_t);
  hipLaunchKernelGGL(clear_words_kernel, dim3((uint32_t)std::min<uint64_t>(1024, (words + 255) / 256)), dim3(256), 0,
                     st, reinterpret_cast<uint32_t *>(acc), words);
  return hipGetLastError();
}

// Both passes of a comparison, on device buffers the caller provides (acc:
// n_groups accumulators; active: n_groups bytes), leaving the accumulators
// in `host`.  The first pass marks the groups that differ in any bit; when
// none does (a correct switch), every figure is 0 and the second pass does
// not run.  Otherwise the marked groups are compared again with every figure.
hipError_t compare_passes(const emrs_plan *plan, const CompareJob &job, const DevSeg *table, const uint32_t *grp,
                          const uint64_t *tab, GroupAcc *acc, uint8_t *active, uint32_t n_groups, hipStream_t st,
                          std::vector<GroupAcc> &host) {
  const size_t acc_bytes = (size_t)n_groups * sizeof(GroupAcc);
  hipError_t e = clear_acc(acc, n_groups, st);
  if (e == hipSuccess) e = compare_launch(plan, job, table, grp, tab, acc, nullptr, st);
  if (e == hipSuccess) e = hipMemcpyAsync(host.data(), acc, acc_bytes, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) return e;
  std::vector<uint8_t> mark(n_groups, 0);
  bool any = false;
  for (uint32_t g = 0; g < n_groups; ++g)
    if (host[g].mismatches) mark[g] = 1, any = true;
  if (!any) return hipSuccess;
  e = hipMemcpyAsync(active, mark.data(), n_groups, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = clear_acc(acc, n_groups, st);
  if (e == hipSuccess) e = compare_launch(plan, job, table, grp, tab, acc, active, st);
  if (e == hipSuccess) e = hipMemcpyAsync(host.data(), acc, acc_bytes, hipMemcpyDeviceToHost, st);
  const hipError_t se = hipStreamSynchronize(st);  // `mark` is read by the copy above
  return e == hipSuccess ? se : e;
}

void compare_finish(const std::vector<GroupAcc> &host, emrs_compare_stats *stats) {
  for (size_t g = 0; g < host.size(); ++g) {
    stats[g].mismatches = host[g].mismatches;
    stats[g].nonfinite = host[g].nonfinite;
    stats[g].sum_sq_diff = host[g].sum_sq_diff;
    stats[g].sum_sq_expected = host[g].sum_sq_expected;
    uint32_t ma = host[g].max_abs_bits, mr = host[g].max_rel_bits;
    memcpy(&stats[g].max_abs_diff, &ma, 4);
    memcpy(&stats[g].max_rel_diff, &mr, 4);
  }
}

// Per device: the address of `scratch` (the array's host-side name is not a
// device address), looked up once with that device current, and the mutex
// that serialises the calls sharing it.
std::mutex g_scratch_mu;
std::vector<unsigned char *> g_scratch_ptr;
std::vector<std::unique_ptr<std::mutex>> g_scratch_call_mu;

int scratch_of(int dev, unsigned char **out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(EMRS_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = static_cast<unsigned char *>(p);
  }
  *out = g_scratch_ptr[dev];
  return EMRS_OK;
}

std::mutex *scratch_call_mutex(int dev) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  while ((int)g_scratch_call_mu.size() <= dev) g_scratch_call_mu.emplace_back(new std::mutex);
  return g_scratch_call_mu[dev].get();
}

}  // namespace

extern "C" {

const char *emrs_last_error(void) { return g_last_error.c_str(); }

int emrs_abi_version(void) { return EMRS_ABI_VERSION; }

int emrs_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

int emrs_plan_create(const emrs_segment *segs, uint64_t n_segs, const uint64_t *src_buf_bytes,
                     uint32_t n_src_bufs, const uint64_t *dst_buf_bytes, uint32_t n_dst_bufs,
                     uint32_t flags, emrs_plan **out_plan) {
  g_last_error.clear();
  if (!out_plan) return fail(EMRS_ERR_INVALID_ARGUMENT, "out_plan is NULL");
  *out_plan = nullptr;
  if (n_segs && !segs) return fail(EMRS_ERR_INVALID_ARGUMENT, "segs is NULL");
  if (n_src_bufs > EMRS_MAX_BUFFERS || n_dst_bufs > EMRS_MAX_BUFFERS)
    return fail(EMRS_ERR_TOO_MANY_BUFFERS, "more than EMRS_MAX_BUFFERS buffers on one side");
  if ((n_src_bufs && !src_buf_bytes) || (n_dst_bufs && !dst_buf_bytes))
    return fail(EMRS_ERR_INVALID_ARGUMENT, "buffer size array is NULL");
  if (flags & ~EMRS_PLAN_CHECK_DISJOINT) return fail(EMRS_ERR_INVALID_ARGUMENT, "unknown flags");
  if (n_segs > 0xffffffffull) return fail(EMRS_ERR_INVALID_ARGUMENT, "more than 2^32 - 1 segments");

  Builder bld;
  bld.out.reserve(n_segs);
  uint64_t payload = 0, read = 0;
  std::vector<uint8_t> src_used(n_src_bufs, 0), dst_used(n_dst_bufs, 0);
  for (uint64_t i = 0; i < n_segs; ++i) {
    const emrs_segment &s = segs[i];
    char where[64];
    snprintf(where, sizeof where, "segment %llu: ", (unsigned long long)i);
    const std::string at(where);
    const int lg = log2_of(s.elem_bytes);
    const bool cast = (s.flags & EMRS_SEG_CAST_BF16) != 0;
    const bool zero = (s.flags & EMRS_SEG_ZERO_FILL) != 0;
    const bool dup = (s.flags & EMRS_SEG_DUP) != 0;
    const bool has_aux = cast || dup;
    if (lg < 0) return fail(EMRS_ERR_INVALID_ARGUMENT, at + "elem_bytes must be 1, 2, 4 or 8");
    if ((s.flags & ~(EMRS_SEG_CAST_BF16 | EMRS_SEG_ZERO_FILL | EMRS_SEG_DUP)) || s.reserved)
      return fail(EMRS_ERR_INVALID_ARGUMENT, at + "unknown flags");
    if (cast && dup) return fail(EMRS_ERR_INVALID_ARGUMENT, at + "a segment carries a bf16 image or a duplicate, not both");
    if (cast && s.elem_bytes != 4) return fail(EMRS_ERR_INVALID_ARGUMENT, at + "a bf16 cast needs fp32 elements");
    if (s.src_buf >= n_src_bufs || s.dst_buf >= n_dst_bufs || (has_aux && s.aux_buf >= n_dst_bufs))
      return fail(EMRS_ERR_INVALID_ARGUMENT, at + "buffer id out of range");
    if (s.rows == 0) return fail(EMRS_ERR_INVALID_ARGUMENT, at + "rows must be >= 1");
    if (s.len == 0) continue;
    if (s.rows > 1 && (s.dst_stride < s.len || (has_aux && s.aux_stride < s.len)))
      return fail(EMRS_ERR_INVALID_ARGUMENT, at + "a destination stride < len makes rows overlap");
    if (!zero && extent_end(s.src_off, s.len, s.rows, s.rows > 1 ? s.src_stride : 0, s.elem_bytes) >
                     src_buf_bytes[s.src_buf])
      return fail(EMRS_ERR_OUT_OF_BOUNDS, at + "source range exceeds its buffer");
    if (extent_end(s.dst_off, s.len, s.rows, s.rows > 1 ? s.dst_stride : 0, s.elem_bytes) > dst_buf_bytes[s.dst_buf])
      return fail(EMRS_ERR_OUT_OF_BOUNDS, at + "destination range exceeds its buffer");
    // Bytes per aux element: a bf16 image, or a duplicate of the element.
    const uint64_t aeb = cast ? 2 : (dup ? s.elem_bytes : 0);
    if (has_aux && extent_end(s.aux_off, s.len, s.rows, s.rows > 1 ? s.aux_stride : 0, (uint32_t)aeb) >
                       dst_buf_bytes[s.aux_buf])
      return fail(EMRS_ERR_OUT_OF_BOUNDS, at + (cast ? "bf16 range exceeds its buffer" : "duplicate range exceeds its buffer"));
    if (!zero) read += s.len * s.rows * s.elem_bytes;
    payload += s.len * s.rows * (s.elem_bytes + aeb);
    if (!zero) src_used[s.src_buf] = 1;
    dst_used[s.dst_buf] = 1;
    if (has_aux) dst_used[s.aux_buf] = 1;

    const uint64_t eb = s.elem_bytes;
    bld.cur_origin = (uint32_t)i;
    bld.cur_elem_log2 = (uint8_t)lg;
    // A zero fill has no source: align its phantom source with the destination.
    const uint64_t so = zero ? s.dst_off * eb : s.src_off * eb, dof = s.dst_off * eb, lb = s.len * eb;
    const uint64_t ds = s.rows > 1 ? s.dst_stride * eb : 0, ss = zero ? ds : (s.rows > 1 ? s.src_stride * eb : 0);
    const uint64_t ao = s.aux_off * aeb, as = s.rows > 1 ? s.aux_stride * aeb : 0;
    Aux ax;
    ax.on = has_aux;
    ax.cast = cast;
    ax.dup = dup;
    ax.zero = zero;
    ax.buf = s.aux_buf;
    // Aux bytes per 16-byte unit: 8 for a bf16 image of fp32, 16 for a duplicate.
    const uint64_t avu = has_aux ? 16 * aeb / eb : 16;
    const bool aux_vec_ok = !has_aux || (ao % avu == 0 && as % avu == 0);
    const bool rows1 = s.rows == 1 || (ss == lb && ds == lb && (!has_aux || as == s.len * aeb));
    if (rows1) {
      const uint64_t L = lb * s.rows;  // contiguous bytes
      if (so % 16 == 0 && dof % 16 == 0 && L % 16 == 0 && aux_vec_ok) {
        ax.off = ao / avu;
        bld.emit(s.src_buf, s.dst_buf, 4, so / 16, dof / 16, L / 16, 1, 0, 0, ax);
      } else if (so % 16 == dof % 16 && (!has_aux || (ao % avu) * eb / aeb == so % 16)) {
        // Source, destination and aux reach a 16-byte boundary at the same element.
        const uint64_t head = std::min<uint64_t>((16 - so % 16) % 16, L);
        const uint64_t body = (L - head) / 16 * 16;
        const uint64_t tail = L - head - body;
        const uint64_t aux_head = head * aeb / eb, aux_body = body * aeb / eb;
        ax.off = has_aux ? ao / aeb : 0;
        bld.emit(s.src_buf, s.dst_buf, lg, so / eb, dof / eb, head / eb, 1, 0, 0, ax);
        ax.off = has_aux ? (ao + aux_head) / avu : 0;
        bld.emit(s.src_buf, s.dst_buf, 4, (so + head) / 16, (dof + head) / 16, body / 16, 1, 0, 0, ax);
        ax.off = has_aux ? (ao + aux_head + aux_body) / aeb : 0;
        bld.emit(s.src_buf, s.dst_buf, lg, (so + head + body) / eb, (dof + head + body) / eb, tail / eb, 1, 0, 0, ax);
      } else {
        ax.off = s.aux_off;
        bld.emit(s.src_buf, s.dst_buf, lg, so / eb, s.dst_off, L / eb, 1, 0, 0, ax);
      }
    } else if (so % 16 == 0 && dof % 16 == 0 && lb % 16 == 0 && ss % 16 == 0 && ds % 16 == 0 && aux_vec_ok) {
      ax.off = ao / avu;
      ax.stride = as / avu;
      bld.emit(s.src_buf, s.dst_buf, 4, so / 16, dof / 16, lb / 16, s.rows, ss / 16, ds / 16, ax);
    } else {
      ax.off = s.aux_off;
      ax.stride = s.rows > 1 ? s.aux_stride : 0;
      bld.emit(s.src_buf, s.dst_buf, lg, so / eb, s.dst_off, s.len, s.rows, ss / eb, s.dst_stride, ax);
    }
  }
  if (flags & EMRS_PLAN_CHECK_DISJOINT) {
    int rc = check_disjoint(segs, n_segs);
    if (rc) return rc;
  }

  if (bld.out.size() > 0xffffffffull) return fail(EMRS_ERR_INVALID_ARGUMENT, "plan needs more than 2^32 - 1 device segments");
  emrs_plan *p = new (std::nothrow) emrs_plan;
  if (!p) return fail(EMRS_ERR_INVALID_ARGUMENT, "out of host memory");
  p->segs = std::move(bld.out);
  p->origin = std::move(bld.origin);
  p->n_chunks = bld.chunks;
  make_hint(p->segs, p->n_chunks, &p->hint);
  p->src_bytes.assign(src_buf_bytes, src_buf_bytes + n_src_bufs);
  p->dst_bytes.assign(dst_buf_bytes, dst_buf_bytes + n_dst_bufs);
  p->src_used = std::move(src_used);
  p->dst_used = std::move(dst_used);
  p->stats.n_segments = n_segs;
  p->stats.n_device_segments = p->segs.size();
  p->stats.payload_bytes = payload;
  p->stats.read_bytes = read;
  p->stats.vector_bytes = bld.vec_bytes;
  p->stats.scalar_bytes = bld.scalar_bytes;
  p->stats.n_chunks = bld.chunks;
  p->stats.n_src_bufs = n_src_bufs;
  p->stats.n_dst_bufs = n_dst_bufs;
  *out_plan = p;
  return EMRS_OK;
}

}  // extern "C"

namespace {
template <int L, int U, bool kBuf>
void launch_chunks(bool nt, const ResolvedBases &rb, dim3 grid, hipStream_t st, const DevSeg *table,
                   uint64_t n_chunks, const SegHint &hint, const uint64_t *stab, const uint64_t *dtab,
                   const uint32_t *cseg) {
  const dim3 block(L);
  const uint32_t remap = g_tuning.xcd_remap.load();
  const bool by_xcd = remap == 2 || (remap == 1 && n_chunks >= kXcdRemapMinChunks);
  const uint64_t xcd_share = by_xcd ? n_chunks * (kChunkUnits / (L * U)) / 8 : 0;
  if (nt && rb.table)
    hipLaunchKernelGGL((copy_plan_kernel<true, true, L, U, kBuf>), grid, block, 0, st, table, n_chunks, hint,
                       rb.src, rb.dst, stab, dtab, xcd_share, cseg);
  else if (nt)
    hipLaunchKernelGGL((copy_plan_kernel<true, false, L, U, kBuf>), grid, block, 0, st, table, n_chunks, hint,
                       rb.src, rb.dst, stab, dtab, xcd_share, cseg);
  else if (rb.table)
    hipLaunchKernelGGL((copy_plan_kernel<false, true, L, U, kBuf>), grid, block, 0, st, table, n_chunks, hint,
                       rb.src, rb.dst, stab, dtab, xcd_share, cseg);
  else
    hipLaunchKernelGGL((copy_plan_kernel<false, false, L, U, kBuf>), grid, block, 0, st, table, n_chunks, hint,
                       rb.src, rb.dst, stab, dtab, xcd_share, cseg);
}

// The one-workgroup-per-piece launch for `lanes` lanes of `units` units each.
template <bool kBuf>
void launch_pieces(uint32_t lanes, uint32_t units, bool nt, const ResolvedBases &rb, dim3 grid, hipStream_t st,
                   const DevSeg *table, uint64_t n_chunks, const SegHint &hint, const uint64_t *stab,
                   const uint64_t *dtab, const uint32_t *cseg) {
  switch (lanes * 8 + units) {
    case 64 * 8 + 1: launch_chunks<64, 1, kBuf>(nt, rb, grid, st, table, n_chunks, hint, stab, dtab, cseg); break;
    case 64 * 8 + 2: launch_chunks<64, 2, kBuf>(nt, rb, grid, st, table, n_chunks, hint, stab, dtab, cseg); break;
    case 128 * 8 + 1: launch_chunks<128, 1, kBuf>(nt, rb, grid, st, table, n_chunks, hint, stab, dtab, cseg); break;
    case 128 * 8 + 2: launch_chunks<128, 2, kBuf>(nt, rb, grid, st, table, n_chunks, hint, stab, dtab, cseg); break;
    case 256 * 8 + 1: launch_chunks<256, 1, kBuf>(nt, rb, grid, st, table, n_chunks, hint, stab, dtab, cseg); break;
    default: launch_chunks<64, 4, kBuf>(nt, rb, grid, st, table, n_chunks, hint, stab, dtab, cseg); break;
  }
}
}  // namespace

extern "C" {

int emrs_plan_stats_get(const emrs_plan *plan, emrs_plan_stats *out) {
  if (!plan || !out) return fail(EMRS_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = plan->stats;
  return EMRS_OK;
}

int emrs_plan_prepare(emrs_plan *plan, void *stream) {
  g_last_error.clear();
  if (!plan) return fail(EMRS_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (plan->n_chunks == 0) return EMRS_OK;
  int dev = 0, cus = 0, resident_nt = 0, resident_t = 0;
  int rc = current_device(&dev, &cus, &resident_nt, &resident_t);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if ((rc = refuse_capture(st, "emrs_plan_prepare"))) return rc;
  DevSeg *table = nullptr;
  rc = device_table(plan, dev, st, &table);
  if (rc) return rc;
  if (g_tuning.chunk_index.load() && !g_tuning.persistent.load()) {
    uint32_t *cseg = nullptr;
    rc = chunk_table(plan, dev, st, table, &cseg);
  }
  return rc;
}

int emrs_plan_execute(emrs_plan *plan, void *const *src_bases, void *const *dst_bases,
                      void *stream) {
  g_last_error.clear();
  if (!plan) return fail(EMRS_ERR_INVALID_ARGUMENT, "plan is NULL");
  ResolvedBases rb;
  int rc = resolve_bases(plan, src_bases, dst_bases, &rb);
  if (rc) return rc;
  if (plan->n_chunks == 0) return EMRS_OK;

  int dev = 0, cus = 0, resident_nt = 0, resident_t = 0;
  rc = current_device(&dev, &cus, &resident_nt, &resident_t);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  DevSeg *table = nullptr;
  rc = device_table(plan, dev, st, &table);
  if (rc) return rc;

  const bool nt = g_tuning.nontemporal.load() != 0;
  const uint32_t nseg = (uint32_t)plan->segs.size();
  const dim3 block(kThreads);
  if (!g_tuning.persistent.load()) {
    // One workgroup per piece of lanes * units units, on a grid of at most 65535 rows.
    const uint32_t lanes = g_tuning.lanes.load(), units = g_tuning.units.load();
    const uint64_t n_wg = plan->n_chunks * (kChunkUnits / (lanes * units));
    const uint64_t gx = std::min<uint64_t>(n_wg, std::max<uint64_t>(1ull << 16, (n_wg + kMaxGridY - 1) / kMaxGridY));
    if (gx > 0xffffffffull / lanes) return fail(EMRS_ERR_INVALID_ARGUMENT, "plan has too many chunks for one launch");
    const dim3 grid((uint32_t)gx, (uint32_t)((n_wg + gx - 1) / gx));
    uint64_t *tab = nullptr;
    bool tab_owned = false;
    rc = pointer_table(plan, dev, rb, st, &tab, &tab_owned);
    if (rc) return rc;
    const uint64_t *stab = tab, *dtab = tab ? tab + plan->stats.n_src_bufs : nullptr;
    // The bases of the cached pointer table also have a resolved segment
    // table: no per-workgroup base lookup.
    const ResolvedBases *lb = &rb;
    ResolvedBases flat;
    if (rb.table && !tab_owned) {
      DevSeg *abs = nullptr;
      char *common = nullptr;
      rc = resolved_table(plan, dev, rb, st, &abs, &common);
      if (rc) return rc;
      if (abs) {
        table = abs;
        flat.src.p[0] = flat.dst.p[0] = common;
        lb = &flat;
        stab = dtab = nullptr;
      }
    }
    uint32_t *cseg = nullptr;
    if (g_tuning.chunk_index.load()) {
      rc = chunk_table(plan, dev, st, table, &cseg);
      if (rc) {
        if (tab_owned) (void)hipFreeAsync(tab, st);
        return rc;
      }
    }
    if (cseg && g_tuning.warm_tables.load()) {
      // 16-byte loads over the whole chunk table (its last 1-3 words share a line with the ones
      // before) and every segment descriptor.
      const uint64_t na = plan->n_chunks / 4, nb = (uint64_t)nseg * sizeof(DevSeg) / sizeof(u32x4);
      const uint64_t blocks = std::min<uint64_t>((na + nb + 255) / 256, 4096);
      hipLaunchKernelGGL(warm_tables_kernel, dim3((uint32_t)blocks), dim3(256), 0, st,
                         reinterpret_cast<const u32x4 *>(cseg), na, reinterpret_cast<const u32x4 *>(table), nb);
    }
    if (g_tuning.buffer_ops.load())
      launch_pieces<true>(lanes, units, nt, *lb, grid, st, table, plan->n_chunks, plan->hint, stab, dtab, cseg);
    else
      launch_pieces<false>(lanes, units, nt, *lb, grid, st, table, plan->n_chunks, plan->hint, stab, dtab, cseg);
    hipError_t le = hipGetLastError();
    if (tab_owned) (void)hipFreeAsync(tab, st);
    if (le != hipSuccess) return hip_fail(le, "copy_plan_kernel launch");
    return note_launch(plan, dev, st);
  }

  // Persistent grid.  A run of N counts N steps of kUnroll chunks.
  const uint32_t bpc = g_tuning.blocks_per_cu.load();
  const uint64_t max_blocks = (uint64_t)cus * (bpc ? bpc : (uint32_t)(nt ? resident_nt : resident_t));
  uint64_t blocks = std::min<uint64_t>(plan->n_chunks, max_blocks);
  uint32_t run = g_tuning.run.load() * kUnroll;
  const bool remap = g_tuning.xcd_remap.load() != 0;
  if (run) {
    // Round-robin runs: at most a quarter of each workgroup's share, so that
    // small plans still spread over the whole grid.
    run = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(run, plan->n_chunks / (blocks * 4)));
    blocks = std::min<uint64_t>(blocks, (plan->n_chunks + run - 1) / run);
  }
  if (remap) blocks = (blocks + 7) / 8 * 8;
  const uint64_t cpb = (plan->n_chunks + blocks - 1) / blocks;
  if (!remap && !run) blocks = (plan->n_chunks + cpb - 1) / cpb;
  const uint32_t xcd_stride = remap ? (uint32_t)(blocks / 8) : 0;
  uint64_t *tab = nullptr;
  bool tab_owned = false;
  rc = pointer_table(plan, dev, rb, st, &tab, &tab_owned);
  if (rc) return rc;
  const uint64_t *stab = tab, *dtab = tab ? tab + plan->stats.n_src_bufs : nullptr;
  const dim3 grid((uint32_t)blocks);
  if (nt && rb.table)
    hipLaunchKernelGGL((copy_plan_persistent_kernel<true, true>), grid, block, 0, st, table, nseg, plan->n_chunks,
                       cpb, xcd_stride, run, rb.src, rb.dst, stab, dtab);
  else if (nt)
    hipLaunchKernelGGL((copy_plan_persistent_kernel<true, false>), grid, block, 0, st, table, nseg, plan->n_chunks,
                       cpb, xcd_stride, run, rb.src, rb.dst, stab, dtab);
  else if (rb.table)
    hipLaunchKernelGGL((copy_plan_persistent_kernel<false, true>), grid, block, 0, st, table, nseg, plan->n_chunks,
                       cpb, xcd_stride, run, rb.src, rb.dst, stab, dtab);
  else
    hipLaunchKernelGGL((copy_plan_persistent_kernel<false, false>), grid, block, 0, st, table, nseg, plan->n_chunks,
                       cpb, xcd_stride, run, rb.src, rb.dst, stab, dtab);
  hipError_t le = hipGetLastError();
  if (tab_owned) (void)hipFreeAsync(tab, st);
  if (le != hipSuccess) return hip_fail(le, "copy_plan_persistent_kernel launch");
  return note_launch(plan, dev, st);
}

int emrs_plan_compare(emrs_plan *plan, void *const *src_bases, void *const *dst_bases, const uint32_t *groups,
                      const uint32_t *aux_groups, uint32_t n_groups, emrs_compare_stats *stats, void *stream) {
  g_last_error.clear();
  CompareJob job;
  int rc = compare_setup(plan, src_bases, dst_bases, groups, aux_groups, n_groups, stats, &job);
  if (rc || plan->n_chunks == 0) return rc;
  int dev = 0;
  rc = compare_device(&job, &dev);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // The comparison allocates its accumulators and waits for the stream.
  rc = refuse_capture(st, "emrs_plan_compare");
  if (rc) return rc;
  DevSeg *table = nullptr;
  rc = device_table(plan, dev, st, &table);
  if (rc) return rc;

  const size_t acc_bytes = align256((size_t)n_groups * sizeof(GroupAcc));
  const size_t grp_bytes = align256(job.g_host.size() * sizeof(uint32_t));
  char *buf = nullptr;
  hipError_t e = hipMalloc(&buf, acc_bytes + grp_bytes + n_groups);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc(compare buffers)");
  GroupAcc *acc = reinterpret_cast<GroupAcc *>(buf);
  uint32_t *grp = reinterpret_cast<uint32_t *>(buf + acc_bytes);
  uint8_t *active = reinterpret_cast<uint8_t *>(buf + acc_bytes + grp_bytes);
  std::vector<GroupAcc> host(n_groups);
  e = hipMemcpyAsync(grp, job.g_host.data(), job.g_host.size() * sizeof(uint32_t), hipMemcpyHostToDevice, st);
  uint64_t *tab = nullptr;
  bool tab_owned = false;
  int table_rc = EMRS_OK;  // a pointer-table failure keeps its own message
  if (e == hipSuccess) table_rc = pointer_table(plan, dev, job.rb, st, &tab, &tab_owned);
  if (e == hipSuccess && table_rc == EMRS_OK) {
    uint32_t *cseg = nullptr;  // null when it does not fit: the first pass then runs as a persistent grid
    table_rc = chunk_table(plan, dev, st, table, &cseg);
    job.cseg = cseg;
  }
  if (e == hipSuccess && table_rc == EMRS_OK)
    e = compare_passes(plan, job, table, grp, tab, acc, active, n_groups, st, host);
  if (tab_owned) (void)hipFreeAsync(tab, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  (void)hipFree(buf);
  if (table_rc != EMRS_OK) return table_rc;
  if (e != hipSuccess) return hip_fail(e, "compare_plan_kernel");
  compare_finish(host, stats);
  return EMRS_OK;
}

int emrs_plan_compare_static(emrs_plan *plan, void *const *src_bases, void *const *dst_bases,
                             const uint32_t *groups, const uint32_t *aux_groups, uint32_t n_groups,
                             emrs_compare_stats *stats, void *stream) {
  g_last_error.clear();
  CompareJob job;
  int rc = compare_setup(plan, src_bases, dst_bases, groups, aux_groups, n_groups, stats, &job);
  if (rc || plan->n_chunks == 0) return rc;
  // Everything the kernel reads or writes beyond the caller's buffers lives in `scratch`, in
  // 256-byte aligned regions: accumulators, group ids, the segment table, the pointer table.
  const size_t nd = plan->segs.size();
  const size_t acc_bytes = align256((size_t)n_groups * sizeof(GroupAcc));
  const size_t grp_bytes = align256(job.g_host.size() * sizeof(uint32_t));
  const size_t seg_bytes = align256(nd * sizeof(DevSeg));
  const size_t ptr_bytes = job.rb.table ? align256(job.rb.ptrs.size() * sizeof(uint64_t)) : 0;
  const size_t act_bytes = align256(n_groups);
  const size_t need = acc_bytes + grp_bytes + seg_bytes + ptr_bytes + act_bytes;
  if (need > EMRS_STATIC_SCRATCH_BYTES) {
    char msg[200];
    snprintf(msg, sizeof msg,
             "the comparison needs %zu bytes of scratch (%zu segments, %u groups); the allocation-free "
             "entry point holds at most %u: use emrs_plan_compare",
             need, nd, n_groups, (unsigned)EMRS_STATIC_SCRATCH_BYTES);
    return fail(EMRS_ERR_TOO_LARGE, msg);
  }
  int dev = 0;
  rc = compare_device(&job, &dev);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = refuse_capture(st, "emrs_plan_compare_static");  // it waits for the stream
  if (rc) return rc;
  unsigned char *base = nullptr;
  rc = scratch_of(dev, &base);
  if (rc) return rc;

  // One call at a time per device: the array is shared by every call on it.
  std::lock_guard<std::mutex> lk(*scratch_call_mutex(dev));
  GroupAcc *acc = reinterpret_cast<GroupAcc *>(base);
  uint32_t *grp = reinterpret_cast<uint32_t *>(base + acc_bytes);
  DevSeg *table = reinterpret_cast<DevSeg *>(base + acc_bytes + grp_bytes);
  uint64_t *tab = job.rb.table ? reinterpret_cast<uint64_t *>(base + acc_bytes + grp_bytes + seg_bytes) : nullptr;
  uint8_t *active = base + acc_bytes + grp_bytes + seg_bytes + ptr_bytes;
  // The previous call's accumulators are still there: compare_passes clears them with a kernel.
  hipError_t e =
      hipMemcpyAsync(grp, job.g_host.data(), job.g_host.size() * sizeof(uint32_t), hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipMemcpyAsync(table, plan->segs.data(), nd * sizeof(DevSeg), hipMemcpyHostToDevice, st);
  if (e == hipSuccess && tab)
    e = hipMemcpyAsync(tab, job.rb.ptrs.data(), job.rb.ptrs.size() * sizeof(uint64_t), hipMemcpyHostToDevice, st);
  std::vector<GroupAcc> host(n_groups);
  job.cseg = existing_chunk_table(plan, dev);  // never built here: that would allocate
  if (e == hipSuccess) e = compare_passes(plan, job, table, grp, tab, acc, active, n_groups, st, host);
  // The host copies above read job's and plan's vectors: wait before they can go.
  const hipError_t se = hipStreamSynchronize(st);
  if (e == hipSuccess) e = se;
  if (e != hipSuccess) return hip_fail(e, "compare_plan_kernel (static scratch)");
  compare_finish(host, stats);
  return EMRS_OK;
}

int emrs_plan_destroy(emrs_plan *plan) {
  if (!plan) return EMRS_OK;
  int prev = 0;
  (void)hipGetDevice(&prev);
  const size_t n_dev = std::max({plan->dev_tables.size(), plan->ptr_tables.size(), plan->abs_tables.size(),
                                  plan->chunk_tables.size(), plan->launch_events.size()});
  for (size_t d = 0; d < n_dev; ++d) {
    DevSeg *segs = d < plan->dev_tables.size() ? plan->dev_tables[d] : nullptr;
    uint64_t *ptrs = d < plan->ptr_tables.size() ? plan->ptr_tables[d] : nullptr;
    DevSeg *abs = d < plan->abs_tables.size() ? plan->abs_tables[d] : nullptr;
    uint32_t *chunks = d < plan->chunk_tables.size() ? plan->chunk_tables[d] : nullptr;
    std::vector<hipEvent_t> evs = d < plan->launch_events.size() ? plan->launch_events[d] : std::vector<hipEvent_t>();
    if (!(segs || ptrs || abs || chunks || !evs.empty())) continue;
    (void)hipSetDevice((int)d);
    // A graph may replay the plan's launches at any time: only a drained device is safe.
    if (plan->captured) (void)hipDeviceSynchronize();
    // The tables are freed on the library's stream after the launches that read them, and only
    // after those: work on other streams is not waited for, and the host does not block.
    hipStream_t fs = free_stream((int)d);
    if (!fs) {
      (void)hipDeviceSynchronize();
    } else {
      for (hipEvent_t ev : evs) (void)hipStreamWaitEvent(fs, ev, 0);
    }
    for (hipEvent_t ev : evs) (void)hipEventDestroy(ev);
    for (void *t : {static_cast<void *>(segs), static_cast<void *>(ptrs), static_cast<void *>(abs),
                    static_cast<void *>(chunks)})
      if (t) (void)hipFreeAsync(t, fs);
  }
  (void)hipSetDevice(prev);
  delete plan;
  return EMRS_OK;
}

int emrs_get_tuning(emrs_tuning *out) {
  if (!out) return fail(EMRS_ERR_INVALID_ARGUMENT, "NULL argument");
  out->blocks_per_cu = g_tuning.blocks_per_cu.load();
  out->nontemporal = g_tuning.nontemporal.load();
  out->xcd_remap = g_tuning.xcd_remap.load();
  out->run = g_tuning.run.load();
  out->persistent = g_tuning.persistent.load();
  out->lanes = g_tuning.lanes.load();
  out->units = g_tuning.units.load();
  out->buffer_ops = g_tuning.buffer_ops.load();
  out->chunk_index = g_tuning.chunk_index.load();
  out->warm_tables = g_tuning.warm_tables.load();
  return EMRS_OK;
}

int emrs_set_tuning(const emrs_tuning *t) {
  if (!t) return fail(EMRS_ERR_INVALID_ARGUMENT, "NULL argument");
  if (t->blocks_per_cu > 64) return fail(EMRS_ERR_INVALID_ARGUMENT, "blocks_per_cu must be in [0, 64]");
  if (t->run > (1u << 20)) return fail(EMRS_ERR_INVALID_ARGUMENT, "run must be in [0, 2^20]");
  if (t->xcd_remap > 2) return fail(EMRS_ERR_INVALID_ARGUMENT, "xcd_remap must be 0, 1 or 2");
  if (t->lanes != 0 && t->lanes != 64 && t->lanes != 128 && t->lanes != 256)
    return fail(EMRS_ERR_INVALID_ARGUMENT, "lanes must be 0, 64, 128 or 256");
  const uint32_t lanes = t->lanes ? t->lanes : 64;
  // 0 keeps the pre-existing meaning: one chunk of 256 units per workgroup.
  const uint32_t units = t->units ? t->units : kChunkUnits / lanes;
  if (units != 1 && units != 2 && units != 4) return fail(EMRS_ERR_INVALID_ARGUMENT, "units must be 0, 1, 2 or 4");
  if (kChunkUnits % (lanes * units)) return fail(EMRS_ERR_INVALID_ARGUMENT, "lanes * units must divide 256");
  g_tuning.blocks_per_cu.store(t->blocks_per_cu);
  g_tuning.nontemporal.store(t->nontemporal ? 1 : 0);
  g_tuning.xcd_remap.store(t->xcd_remap);
  g_tuning.run.store(t->run);
  g_tuning.persistent.store(t->persistent ? 1 : 0);
  g_tuning.lanes.store(lanes);
  g_tuning.units.store(units);
  g_tuning.buffer_ops.store(t->buffer_ops ? 1 : 0);
  g_tuning.chunk_index.store(t->chunk_index ? 1 : 0);
  g_tuning.warm_tables.store(t->warm_tables ? 1 : 0);
  return EMRS_OK;
}

}  // extern "C"
