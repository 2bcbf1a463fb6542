// Synthetic optimizer-state generator and on-device verifier for the reshard repack.
//
// Each value is a pure function of (seed, parameter id, kind, full flat
// index), so any shard of any layout can be produced or checked on its own.
// The bits are produced with integer mixing and a single correctly rounded
// fp32 multiply, which host code reproduces exactly:
//   stream key  k = mix64(mix64(seed + G) + (4 * param_id + stream + 1) * G)
//   draw        h = mix64(k + (index + 1) * G)          (G = 0x9E3779B97F4A7C15)
//   normal      s = sum of the four 16-bit lanes of h - 131070     (|s| < 2^18)
//   value       v = float(s) * scale[stream]                  (one fp32 rounding)
// mix64 is the splitmix64 finaliser (Steele, Lea & Flood, OOPSLA 2014).
// Streams: 0 param (rounded to bf16, nearest-even), 1 exp_avg, 2 exp_avg_sq
// (absolute value).  The fp32 main weight is the exact upcast of the bf16
// param, so casting main back to bf16 reproduces the param bit for bit.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "emrs.h"
#include "internal.h"

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;
constexpr int kThreads = 256;
constexpr uint64_t kChunk = 4096;  // elements per work chunk

// fp32 bit patterns of sigma / 37837.227 (std of the 4-lane sum).
constexpr uint32_t kScaleBits[3] = {0x350de3bdu, 0x32e305fbu, 0x2de878d0u};

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t stream_key(uint64_t seed, uint32_t param_id, uint32_t stream) {
  return mix64(mix64(seed + kGamma) + (4ull * param_id + stream + 1) * kGamma);
}

struct DevPiece {
  uint64_t buf_off, len, local_start, local_cols, full_cols, band_rows, row_off, row_off2, col_off;
  uint64_t chunk_begin;
  uint64_t key;
  uint32_t buf, kind;
};

// Buffers of a synthetic fill or check, passed by value in kernel arguments
// (which are limited to a few KB).
constexpr uint32_t kSynthBuffers = 128;

struct SynthBases {
  char *p[kSynthBuffers];
};
static_assert(sizeof(SynthBases) <= 1024, "SynthBases travels in kernel arguments");

__device__ __forceinline__ uint32_t synth_bits(const DevPiece &pc, float scale, uint64_t i) {
  const uint64_t li = pc.local_start + i;
  const uint64_t r = li / pc.local_cols;
  const uint64_t c = li - r * pc.local_cols;
  const uint64_t row = (pc.band_rows == 0 || r < pc.band_rows) ? r + pc.row_off : r - pc.band_rows + pc.row_off2;
  const uint64_t f = row * pc.full_cols + c + pc.col_off;
  const uint64_t h = mix64(pc.key + (f + 1) * kGamma);
  const int32_t s = (int32_t)((h & 0xffff) + ((h >> 16) & 0xffff) + ((h >> 32) & 0xffff) + (h >> 48)) - 131070;
  float v = __fmul_rn((float)s, scale);
  uint32_t bits = __float_as_uint(v);
  if (pc.kind == 3) bits &= 0x7fffffffu;
  if (pc.kind <= 1) {
    const uint32_t bf = (bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16;  // round to nearest even
    bits = pc.kind == 0 ? bf : (bf << 16);
  }
  return bits;
}

__device__ __forceinline__ uint32_t find_piece(const DevPiece *pcs, uint32_t n, uint64_t c) {
  uint32_t lo = 0, hi = n - 1;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (pcs[mid].chunk_begin <= c) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

__global__ __launch_bounds__(kThreads) void synth_fill_kernel(const DevPiece *__restrict__ pcs, uint32_t n,
                                                              uint64_t n_chunks, SynthBases bases,
                                                              float s0, float s1, float s2) {
  for (uint64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
    const uint32_t pi = find_piece(pcs, n, c);
    const DevPiece pc = pcs[pi];
    const float scale = pc.kind <= 1 ? s0 : (pc.kind == 2 ? s1 : s2);
    const uint64_t e0 = (c - pc.chunk_begin) * kChunk;
    const uint64_t e1 = min(e0 + kChunk, pc.len);
    for (uint64_t i = e0 + threadIdx.x; i < e1; i += kThreads) {
      const uint32_t bits = synth_bits(pc, scale, i);
      if (pc.kind == 0)
        reinterpret_cast<uint16_t *>(bases.p[pc.buf])[pc.buf_off + i] = (uint16_t)bits;
      else
        reinterpret_cast<uint32_t *>(bases.p[pc.buf])[pc.buf_off + i] = bits;
    }
  }
}

__global__ __launch_bounds__(kThreads) void synth_verify_kernel(const DevPiece *__restrict__ pcs, uint32_t n,
                                                                uint64_t n_chunks, SynthBases bases,
                                                                float s0, float s1, float s2,
                                                                unsigned long long *counters) {
  unsigned long long bad = 0;
  unsigned long long first = ~0ull;
  for (uint64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
    const uint32_t pi = find_piece(pcs, n, c);
    const DevPiece pc = pcs[pi];
    const float scale = pc.kind <= 1 ? s0 : (pc.kind == 2 ? s1 : s2);
    const uint64_t e0 = (c - pc.chunk_begin) * kChunk;
    const uint64_t e1 = min(e0 + kChunk, pc.len);
    for (uint64_t i = e0 + threadIdx.x; i < e1; i += kThreads) {
      const uint32_t want = synth_bits(pc, scale, i);
      uint32_t got;
      if (pc.kind == 0)
        got = reinterpret_cast<const uint16_t *>(bases.p[pc.buf])[pc.buf_off + i];
      else
        got = reinterpret_cast<const uint32_t *>(bases.p[pc.buf])[pc.buf_off + i];
      if (got != want) {
        ++bad;
        const unsigned long long tag = ((unsigned long long)pi << 40) | i;
        first = tag < first ? tag : first;
      }
    }
  }
  if (bad) {
    atomicAdd(&counters[0], bad);
    atomicMin(&counters[1], first);
  }
}

int sfail(int code, const std::string &m) { return emrs_internal::fail(code, m); }

int build_pieces(const emrs_piece *pieces, uint64_t n, const uint64_t *buf_bytes, uint32_t n_bufs,
                 uint64_t seed, std::vector<DevPiece> *out, uint64_t *n_chunks) {
  if (n && !pieces) return sfail(EMRS_ERR_INVALID_ARGUMENT, "pieces is NULL");
  if (n_bufs > kSynthBuffers) return sfail(EMRS_ERR_TOO_MANY_BUFFERS, "more than 128 buffers");
  if (n_bufs && !buf_bytes) return sfail(EMRS_ERR_INVALID_ARGUMENT, "buf_bytes is NULL");
  if (n >= (1ull << 24)) return sfail(EMRS_ERR_INVALID_ARGUMENT, "too many pieces");
  uint64_t chunks = 0;
  out->clear();
  out->reserve(n);
  for (uint64_t i = 0; i < n; ++i) {
    const emrs_piece &p = pieces[i];
    if (p.kind > 3) return sfail(EMRS_ERR_INVALID_ARGUMENT, "piece kind must be 0..3");
    if (p.buf >= n_bufs) return sfail(EMRS_ERR_INVALID_ARGUMENT, "piece buffer id out of range");
    if (p.local_cols == 0 || p.full_cols == 0) return sfail(EMRS_ERR_INVALID_ARGUMENT, "zero columns");
    if (p.len == 0) continue;
    const uint64_t eb = p.kind == 0 ? 2 : 4;
    if ((p.buf_off + p.len) * eb > buf_bytes[p.buf])
      return sfail(EMRS_ERR_OUT_OF_BOUNDS, "piece exceeds its buffer");
    DevPiece d{};
    d.buf_off = p.buf_off;
    d.len = p.len;
    d.local_start = p.local_start;
    d.local_cols = p.local_cols;
    d.full_cols = p.full_cols;
    d.band_rows = p.band_rows;
    d.row_off = p.row_off;
    d.row_off2 = p.row_off2;
    d.col_off = p.col_off;
    d.chunk_begin = chunks;
    d.key = stream_key(seed, p.param_id, p.kind <= 1 ? 0 : p.kind - 1);
    d.buf = p.buf;
    d.kind = p.kind;
    chunks += (p.len + kChunk - 1) / kChunk;
    out->push_back(d);
  }
  *n_chunks = chunks;
  return EMRS_OK;
}

float bits_to_float(uint32_t b) {
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

int launch(bool verify, const emrs_piece *pieces, uint64_t n, void *const *bases,
           const uint64_t *buf_bytes, uint32_t n_bufs, uint64_t seed, void *stream,
           uint64_t *mismatches, uint64_t *first_bad) {
  emrs_internal::clear_error();
  std::vector<DevPiece> dp;
  uint64_t n_chunks = 0;
  int rc = build_pieces(pieces, n, buf_bytes, n_bufs, seed, &dp, &n_chunks);
  if (rc) return rc;
  if (mismatches) *mismatches = 0;
  if (first_bad) *first_bad = ~0ull;
  if (dp.empty()) return EMRS_OK;
  SynthBases sb{};
  for (uint32_t i = 0; i < n_bufs; ++i) sb.p[i] = static_cast<char *>(bases[i]);
  int dev_count = 0;
  if (hipGetDeviceCount(&dev_count) != hipSuccess || dev_count == 0) {
    (void)hipGetLastError();
    return sfail(EMRS_ERR_NO_DEVICE, "no HIP device is visible");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  DevPiece *d_pcs = nullptr;
  unsigned long long *d_cnt = nullptr;
  hipError_t e = hipMalloc(&d_pcs, dp.size() * sizeof(DevPiece));
  if (e != hipSuccess) return sfail(EMRS_ERR_HIP, std::string("hipMalloc: ") + hipGetErrorString(e));
  e = hipMemcpyAsync(d_pcs, dp.data(), dp.size() * sizeof(DevPiece), hipMemcpyHostToDevice, st);
  if (e == hipSuccess && verify) {
    e = hipMalloc(&d_cnt, 2 * sizeof(unsigned long long));
    if (e == hipSuccess) {
      const unsigned long long init[2] = {0ull, ~0ull};
      e = hipMemcpyAsync(d_cnt, init, sizeof init, hipMemcpyHostToDevice, st);
    }
  }
  const uint32_t blocks = (uint32_t)std::min<uint64_t>(n_chunks, 8192);
  const float s0 = bits_to_float(kScaleBits[0]), s1 = bits_to_float(kScaleBits[1]),
              s2 = bits_to_float(kScaleBits[2]);
  if (e == hipSuccess) {
    if (verify)
      hipLaunchKernelGGL(synth_verify_kernel, dim3(blocks), dim3(kThreads), 0, st, d_pcs,
                         (uint32_t)dp.size(), n_chunks, sb, s0, s1, s2, d_cnt);
    else
      hipLaunchKernelGGL(synth_fill_kernel, dim3(blocks), dim3(kThreads), 0, st, d_pcs,
                         (uint32_t)dp.size(), n_chunks, sb, s0, s1, s2);
    e = hipGetLastError();
  }
  unsigned long long host_cnt[2] = {0ull, ~0ull};
  if (e == hipSuccess && verify) e = hipMemcpyAsync(host_cnt, d_cnt, sizeof host_cnt, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  const hipError_t e_work = e;
  if (d_cnt) (void)hipFree(d_cnt);
  (void)hipFree(d_pcs);
  if (e_work != hipSuccess)
    return sfail(EMRS_ERR_HIP, std::string(verify ? "synth verify: " : "synth fill: ") + hipGetErrorString(e_work));
  if (verify) {
    *mismatches = host_cnt[0];
    *first_bad = host_cnt[1];
  }
  return EMRS_OK;
}

}  // namespace

namespace {

// XOR of every 32-bit word of a buffer: the plain read rate of the device.
// One-wavefront workgroups, eight per CU, each with four 16-byte non-temporal
// loads in flight per lane over 4 KB pieces dealt out grid-stride; one atomic
// per workgroup at the end.  Timed on 32-72 GiB buffers, this shape read at
// 7.1-7.3 TB/s where 256-lane workgroups with eight loads per lane, five per
// CU, read at 6.7-6.8 TB/s; 16 or 32 workgroups per CU read slower
// (6.3-6.4 TB/s), as did 128 or 256 lanes with four loads each (6.7-6.8).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kXorLanes = 64;
constexpr int kXorUnroll = 4;
constexpr int kXorBlocksPerCu = 8;
constexpr uint64_t kXorPiece = (uint64_t)kXorLanes * kXorUnroll;   // units per workgroup step

__global__ __launch_bounds__(kXorLanes) void xor_checksum_kernel(const u32x4 *__restrict__ p, uint64_t n_units,
                                                                 uint32_t *__restrict__ out) {
  uint32_t acc = 0;
  const uint64_t step = (uint64_t)gridDim.x * kXorPiece;
  for (uint64_t base = (uint64_t)blockIdx.x * kXorPiece; base < n_units; base += step) {
    u32x4 v[kXorUnroll];
#pragma unroll
    for (int j = 0; j < kXorUnroll; ++j) {
      const uint64_t i = base + (uint64_t)j * kXorLanes + threadIdx.x;
      v[j] = i < n_units ? __builtin_nontemporal_load(p + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < kXorUnroll; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  for (int off = 32; off > 0; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, 64);
  if (threadIdx.x == 0 && acc) atomicXor(out, acc);
}

}  // namespace

extern "C" int emrs_xor_checksum(const void *p, uint64_t bytes, uint32_t *out, void *stream) {
  emrs_internal::clear_error();
  if (!out || (bytes && !p)) return sfail(EMRS_ERR_INVALID_ARGUMENT, "NULL argument");
  if (reinterpret_cast<uintptr_t>(p) % 16 || bytes % 16)
    return sfail(EMRS_ERR_MISALIGNED, "the buffer and its size must be multiples of 16 bytes");
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return sfail(EMRS_ERR_NO_DEVICE, "no HIP device is visible");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  e = hipMemsetAsync(out, 0, sizeof(uint32_t), st);
  if (e != hipSuccess) return sfail(EMRS_ERR_HIP, std::string("hipMemsetAsync: ") + hipGetErrorString(e));
  const uint64_t n_units = bytes / 16;
  if (n_units == 0) return EMRS_OK;
  const uint64_t blocks =
      std::min<uint64_t>((n_units + kXorPiece - 1) / kXorPiece, (uint64_t)std::max(cus, 1) * kXorBlocksPerCu);
  hipLaunchKernelGGL(xor_checksum_kernel, dim3((uint32_t)blocks), dim3(kXorLanes), 0, st,
                     static_cast<const u32x4 *>(p), n_units, out);
  e = hipGetLastError();
  if (e != hipSuccess) return sfail(EMRS_ERR_HIP, std::string("xor_checksum_kernel launch: ") + hipGetErrorString(e));
  return EMRS_OK;
}

extern "C" int emrs_synth_fill(const emrs_piece *pieces, uint64_t n_pieces, void *const *bases,
                               const uint64_t *buf_bytes, uint32_t n_bufs, uint64_t seed, void *stream) {
  return launch(false, pieces, n_pieces, bases, buf_bytes, n_bufs, seed, stream, nullptr, nullptr);
}

extern "C" int emrs_synth_verify(const emrs_piece *pieces, uint64_t n_pieces, void *const *bases,
                                 const uint64_t *buf_bytes, uint32_t n_bufs, uint64_t seed, void *stream,
                                 uint64_t *mismatches, uint64_t *first_bad) {
  if (!mismatches || !first_bad) return sfail(EMRS_ERR_INVALID_ARGUMENT, "NULL output pointer");
  return launch(true, pieces, n_pieces, bases, buf_bytes, n_bufs, seed, stream, mismatches, first_bad);
}
