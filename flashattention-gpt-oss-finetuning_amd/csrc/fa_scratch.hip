// fa_scratch.hip - fa_bwd_scratch: the backward without a caller-supplied workspace.
//
// The backward kernels keep row statistics and partial sums in a workspace (delta, sink-key
// partials, learned-sink partials; fa_bwd_workspace_bytes).  fa_bwd_scratch gives them this
// library's own device buffer instead, a file-scope array of FA_SCRATCH_BYTES bytes that every
// GPU the library runs on holds until the process ends, so the call allocates nothing.  Its
// address on a device is looked up once, on that device's first call, with the device current;
// host code uses only that address (the array's name is a host-side stand-in).
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "../../include/fa_gfx950.h"

namespace {

static __device__ __align__(256) unsigned char scratch[FA_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

// The device address of `scratch` on the current device (NULL on error).
void* scratch_ptr(int dev) {
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (!p) {
    void* q = nullptr;
    if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return nullptr;
    p = q;
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  return p;
}

}  // namespace

extern "C" int fa_bwd_scratch(const fa_bwd_params* p, void* stream) {
  const int rc = fa_check_bwd(p);
  if (rc != FA_OK) return rc;
  const size_t need = fa_bwd_workspace_bytes(p->batch, p->heads_q, p->heads_kv, p->seqlen, p->head_dim, p->window,
                                             p->sink);
  if (need > size_t(FA_SCRATCH_BYTES)) return FA_ERR_SCRATCH;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FA_ERR_LAUNCH;
  void* ws = scratch_ptr(dev);
  if (!ws) return FA_ERR_LAUNCH;
  // the kernels need no zeroed workspace: every value they read there is written first
  return fa_bwd(p, ws, size_t(FA_SCRATCH_BYTES), stream);
}
