/*
 * py_hip.c - the engine's Python FFI library (py/csrc/libthvm.m, compiled
 * where it lies: the engine, its CPU backend, nn and the py_* exports of
 * py/csrc/libthvm.m:52-215) with the HIP backend as a device.
 *
 * TEST INFRASTRUCTURE. Built by `make -C oracle ref` into
 * oracle/_ref/libthvm_py.so with -Dthvm_init=thvm_init_engine; driven over
 * ctypes by tests/test_gpu_pyffi.py.
 *
 * The engine's thvm_init gets the "hip" branch a maintainer adds to it
 * (tests/live/hip_init.h). py_init_hip(path) loads libthvm_hip.so and then
 * makes exactly the engine's own py_init call for device "hip" (py_init,
 * py/csrc/libthvm.m:52-56, is thvm_init(device) after a Metal-only path
 * setup): thvm_init("hip") registers hip_backend as the default device, or
 * stays on the CPU when the backend's init fails. Every other py_* call is
 * the engine's own, unchanged; py_free reaches the backend's shutdown
 * through thvm_free.
 */
#include "libthvm.m"

#undef thvm_init
#include "hip_init.h"

__attribute__((visibility("default")))
TinyHVM *py_init_hip(const char *lib_path) {
    if (hip_backend_load(lib_path, 1) != 0) return NULL;
    return thvm_init("hip");
}

/* the engine context's default device (0 cpu, 2 hip) */
__attribute__((visibility("default")))
u32 py_default_device(TinyHVM *ctx) { return ctx ? ctx->default_device : 0xFFFFFFFFu; }
