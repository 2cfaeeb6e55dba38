// libsolvedelta_noalloc.so: sd_fwd_noalloc, the forward of libsolvedelta_hip.so
// with its workspace in a file-scope device array instead of a caller buffer.
//
// The array lives in this library only, so a process that never loads it (every
// training or autograd user of libsolvedelta_hip.so) carries no static device
// memory; a process that loads it holds SD_NOALLOC_SCRATCH_BYTES on each GPU it
// calls it on, from module load to process end.  The kernels are the main
// library's: this file calls its sd_fwd_split with the two regions carved out of
// the array.
#include <hip/hip_runtime.h>
#include <mutex>
#include "../../../include/solvedelta.h"
#include "../../../include/solvedelta_noalloc.h"

namespace {

// The forward workspace of callers that cannot allocate.  Host code reaches it
// only through the address hipGetSymbolAddress returns for the current device
// (on the host, the array's name is not a device address).
static __device__ __align__(256) unsigned char scratch[SD_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device.
int scratch_for_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return SD_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return SD_ERR_LAUNCH;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return SD_OK;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

extern "C" {

size_t sd_noalloc_scratch_bytes(void) { return SD_NOALLOC_SCRATCH_BYTES; }

int sd_fwd_noalloc(const sd_inputs* in, void* out, float* C_T, float* S_T, void* stream) {
  if (!in || !out) return SD_ERR_ARG;
  if (in->B < 1 || in->T < 1 || in->H < 1 || in->r < 1 || in->V < 1) return SD_ERR_SHAPE;
  const size_t saved = sd_fwd_saved_bytes(in->B, in->T, in->H, in->r, in->V);
  const size_t scratch_b = sd_fwd_scratch_bytes(in->B, in->T, in->H, in->r, in->V);
  if (align256(saved) + scratch_b > SD_NOALLOC_SCRATCH_BYTES) return SD_ERR_WORKSPACE;
  void* base = nullptr;
  const int rc = scratch_for_current_device(&base);
  if (rc) return rc;
  return sd_fwd_split(in, out, C_T, S_T, base, saved, (char*)base + align256(saved), scratch_b,
                      stream);
}

}  // extern "C"
