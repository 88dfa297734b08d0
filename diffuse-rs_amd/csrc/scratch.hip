// scratch.hip -- the fixed device workspace of dr_attention_cached_noalloc.
//
// A file-scope device array that the library never allocates or frees: each
// GPU the library runs on holds one copy from module load until the process
// ends.  Host code must not pass the array's name to a kernel (in host code
// it is a host-side stand-in, not a device address): scratch_init() takes the
// device address of this GPU's copy with hipGetSymbolAddress once per device
// (with that device current), and every kernel argument uses that address.
#include "dr_internal.hpp"

#include <atomic>

namespace dr {
namespace {

constexpr size_t SCRATCH_BYTES = (size_t)64 << 20;
constexpr int MAX_DEVICES = 64;

static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

std::atomic<void*> g_scratch[MAX_DEVICES];

}  // namespace

size_t scratch_bytes() { return SCRATCH_BYTES; }

hipError_t scratch_init(int device) {
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    if (g_scratch[device].load(std::memory_order_acquire)) return hipSuccess;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch[device].store(p, std::memory_order_release);
    return hipSuccess;
}

void* scratch_ptr(int device) {
    if (device < 0 || device >= MAX_DEVICES) return nullptr;
    return g_scratch[device].load(std::memory_order_acquire);
}

}  // namespace dr
