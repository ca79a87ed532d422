// noalloc.hip - the static device workspace of the no-allocation dispatch
// entry point (thvm_hip_dispatch_uop_kernel_noalloc, backend.c).
//
// `scratch` is a file-scope device array: every GPU the library runs on holds
// its own copy, at its own address, from the first lookup until the process
// ends. In host code its name is only a stand-in for the symbol, never a
// device address: the address comes from hipGetSymbolAddress, looked up once
// per device with that device current (at backend init), and only that
// address is handed to kernels and copies. Kernels take it as their workspace
// argument, exactly as they take a pool-allocated workspace in the
// allocating entry point. Nothing here needs to start at zero: every kernel
// that uses it writes a region in full before reading it.
#include <hip/hip_runtime.h>

#include "noalloc.h"

static __device__ __align__(256) unsigned char scratch[THVM_HIP_NOALLOC_SCRATCH_BYTES];

static void *scratch_dev[THVM_NOALLOC_MAX_DEVICES];

extern "C" int thvm_noalloc_scratch_init(int device) {
    if (device < 0 || device >= THVM_NOALLOC_MAX_DEVICES) return -1;
    if (scratch_dev[device]) return 0;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return -1;
    }
    scratch_dev[device] = p;
    return 0;
}

extern "C" void *thvm_noalloc_scratch_ptr(int device) {
    if (device < 0 || device >= THVM_NOALLOC_MAX_DEVICES) return nullptr;
    return scratch_dev[device];
}
