/*
 * py_hip.c - the engine's Python FFI library (py/csrc/libthvm.m, compiled
 * where it lies: the engine, its CPU backend, nn and the py_* exports of
 * py/csrc/libthvm.m:52-215) with the HIP backend as a device.
 *
 * TEST INFRASTRUCTURE. Built by `make -C oracle ref` into
 * oracle/_ref/libthvm_py.so; driven over ctypes by tests/test_gpu_pyffi.py.
 *
 * py_init_hip(path) stands in for the "hip" branch a maintainer adds to
 * thvm_init (src/ctx/init.c:17-35), which this engine version does not have:
 * it loads libthvm_hip.so, initialises its `hip_backend` vtable and registers
 * it as the default device of an engine context, as the Metal branch does
 * for metal_backend. Every other py_* call is the engine's own, unchanged.
 */
#include "libthvm.m"

__attribute__((visibility("default")))
TinyHVM *py_init_hip(const char *lib_path) {
    void *h = dlopen(lib_path, RTLD_NOW | RTLD_GLOBAL);
    if (!h) {
        fprintf(stderr, "py_init_hip: %s\n", dlerror());
        return NULL;
    }
    Backend *hb = (Backend *)dlsym(h, "hip_backend");
    if (!hb || !hb->init || hb->init() != 0) return NULL;
    TinyHVM *ctx = py_init("cpu");
    if (!ctx) return NULL;
    ctx->backends[2] = hb;
    if (ctx->n_backends < 3) ctx->n_backends = 3;
    ctx->default_device = 2;
    return ctx;
}
