// Inter-process hand-off of device buffers: export, open and close.
//
// The reference hands a process's optimizer tensors to its successor with
// one CUDA-IPC handle per tensor storage, packed by _make_cuda_tensor_info
// (elastic_megatron/transfer/ipc_manager.py:23-51) and rebuilt on the other
// side by rebuild_cuda_tensor (:135-155).  Here a state is held in
// allocations of less than 2 GiB each, and each one is exported once.  The
// importer opens the handles and runs the reshard straight from the mapped
// memory: nothing is cloned, and the copy kernel reads the mapped source as it
// reads any other source.
//
// Host code only: no kernel runs here.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "emrs.h"
#include "internal.h"

namespace {

using emrs_internal::fail;

int hip_fail(hipError_t e, const char *what) {
  return fail(EMRS_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

static_assert(sizeof(hipIpcMemHandle_t) == EMRS_IPC_HANDLE_BYTES, "IPC handle size");
static_assert(sizeof(emrs_ipc_buffer) == 96, "emrs_ipc_buffer layout");

// Allocations this process has opened, keyed by handle bytes: opening the same
// allocation again returns the same mapping and only counts another reference.
struct Mapping {
  void *base = nullptr;
  uint64_t refs = 0;
  int device = -1;
};

std::mutex g_mu;
std::map<std::string, Mapping> g_open;  // handle bytes -> mapping
struct Handed {
  std::string key;
  uint64_t count = 0;
};
std::map<uintptr_t, Handed> g_handed;   // pointer handed out -> its allocation, opens not yet closed

}  // namespace

extern "C" {

int emrs_ipc_export(const void *ptr, uint64_t bytes, emrs_ipc_buffer *out) {
  emrs_internal::clear_error();
  if (!ptr || !out) return fail(EMRS_ERR_INVALID_ARGUMENT, "emrs_ipc_export: NULL argument");
  if (bytes == 0) return fail(EMRS_ERR_INVALID_ARGUMENT, "emrs_ipc_export: empty buffer");
  if (reinterpret_cast<uintptr_t>(ptr) % 16)
    return fail(EMRS_ERR_MISALIGNED, "emrs_ipc_export: buffer is not 16-byte aligned");
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, ptr);
  if (e != hipSuccess) return hip_fail(e, "hipPointerGetAttributes");
  if (attr.type != hipMemoryTypeDevice)
    return fail(EMRS_ERR_INVALID_ARGUMENT, "emrs_ipc_export: not device memory");
  void *base = nullptr;
  size_t alloc = 0;
  e = hipMemGetAddressRange(&base, &alloc, const_cast<void *>(ptr));
  if (e != hipSuccess) return hip_fail(e, "hipMemGetAddressRange");
  if (alloc >= EMRS_IPC_MAX_ALLOCATION_BYTES)
    return fail(EMRS_ERR_TOO_LARGE, "emrs_ipc_export: the allocation holding the buffer is " +
                                        std::to_string(alloc) + " bytes; shared allocations must stay under 2 GiB");
  const uint64_t off = reinterpret_cast<uintptr_t>(ptr) - reinterpret_cast<uintptr_t>(base);
  if (off > alloc || bytes > alloc - off)
    return fail(EMRS_ERR_OUT_OF_BOUNDS, "emrs_ipc_export: the buffer runs past its allocation");
  hipIpcMemHandle_t h;
  e = hipIpcGetMemHandle(&h, base);
  if (e != hipSuccess) return hip_fail(e, "hipIpcGetMemHandle");
  std::memset(out, 0, sizeof(*out));
  std::memcpy(out->handle, &h, sizeof(h));
  out->offset = off;
  out->bytes = bytes;
  out->allocation_bytes = alloc;
  out->device = attr.device;
  return EMRS_OK;
}

int emrs_ipc_open(const emrs_ipc_buffer *buf, void **ptr) {
  emrs_internal::clear_error();
  if (!buf || !ptr) return fail(EMRS_ERR_INVALID_ARGUMENT, "emrs_ipc_open: NULL argument");
  *ptr = nullptr;
  if (buf->reserved) return fail(EMRS_ERR_INVALID_ARGUMENT, "emrs_ipc_open: reserved field is not 0");
  // Checked before the driver sees the handle: opening a larger allocation is not supported.
  if (buf->allocation_bytes == 0 || buf->allocation_bytes >= EMRS_IPC_MAX_ALLOCATION_BYTES)
    return fail(EMRS_ERR_TOO_LARGE, "emrs_ipc_open: shared allocations must be non-empty and under 2 GiB");
  if (buf->bytes == 0 || buf->offset > buf->allocation_bytes || buf->bytes > buf->allocation_bytes - buf->offset)
    return fail(EMRS_ERR_OUT_OF_BOUNDS, "emrs_ipc_open: the buffer runs past its allocation");
  if (buf->offset % 16) return fail(EMRS_ERR_MISALIGNED, "emrs_ipc_open: buffer offset is not 16-byte aligned");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  const std::string key(reinterpret_cast<const char *>(buf->handle), EMRS_IPC_HANDLE_BYTES);
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_open.find(key);
  if (it == g_open.end()) {
    hipIpcMemHandle_t h;
    std::memcpy(&h, buf->handle, sizeof(h));
    void *base = nullptr;
    e = hipIpcOpenMemHandle(&base, h, hipIpcMemLazyEnablePeerAccess);
    if (e != hipSuccess) return hip_fail(e, "hipIpcOpenMemHandle");
    it = g_open.emplace(key, Mapping{base, 0, dev}).first;
  } else if (it->second.device != dev) {
    return fail(EMRS_ERR_INVALID_ARGUMENT, "emrs_ipc_open: the allocation is open on another device");
  }
  it->second.refs += 1;
  char *p = static_cast<char *>(it->second.base) + buf->offset;
  Handed &hd = g_handed[reinterpret_cast<uintptr_t>(p)];
  hd.key = key;
  hd.count += 1;
  *ptr = p;
  return EMRS_OK;
}

int emrs_ipc_close(void *ptr) {
  emrs_internal::clear_error();
  std::lock_guard<std::mutex> lk(g_mu);
  auto hp = g_handed.find(reinterpret_cast<uintptr_t>(ptr));
  if (!ptr || hp == g_handed.end())
    return fail(EMRS_ERR_INVALID_ARGUMENT, "emrs_ipc_close: not a pointer emrs_ipc_open returned");
  auto it = g_open.find(hp->second.key);
  Mapping &m = it->second;
  if (m.refs > 1) {  // other opens of the allocation stay valid
    m.refs -= 1;
    if (--hp->second.count == 0) g_handed.erase(hp);
    return EMRS_OK;
  }
  int prev = 0;
  hipError_t e = hipGetDevice(&prev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (prev != m.device && (e = hipSetDevice(m.device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
  e = hipIpcCloseMemHandle(m.base);
  if (prev != m.device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(e, "hipIpcCloseMemHandle");
  g_handed.erase(hp);
  g_open.erase(it);
  return EMRS_OK;
}

int emrs_ipc_open_count(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  return static_cast<int>(g_open.size());
}

}  // extern "C"
