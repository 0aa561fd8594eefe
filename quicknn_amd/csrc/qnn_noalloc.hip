// qnn_noalloc.hip -- the fixed device scratch of qnn_int4_linear_noalloc.
//
// That entry point runs the INT4 projection without allocating device memory:
// its split-K partial sums and per-tile arrival tickets live in `scratch`, a
// file-scope device array of a fixed size.  Each GPU the library runs on holds
// its own copy for the life of the process.
//
// Host code never uses the array's name as a device address (on the host it
// names a host-side stand-in).  noalloc_scratch_init, called by
// qnn_ctx_create with the device current, asks the runtime for the device
// address of this GPU's copy once and keeps it per device; kernels receive
// that address as an argument.
#include <mutex>

#include "qnn_internal.h"

namespace qnn {
namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch_ptr[kMaxDevices] = {};

}  // namespace

void noalloc_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices) fail(QNN_E_ARGUMENT, "device index");
  std::lock_guard<std::mutex> g(g_scratch_lock);
  if (g_scratch_ptr[device]) return;
  void *ptr = nullptr;
  hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  if (!ptr) fail(QNN_E_INVALID_OP, "no device address for the static scratch");
  g_scratch_ptr[device] = ptr;
}

void *noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> g(g_scratch_lock);
  return g_scratch_ptr[device];
}

}  // namespace qnn
