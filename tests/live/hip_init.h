/*
 * hip_init.h - the "hip" branch of thvm_init, as a maintainer adds it to the
 * engine (src/ctx/init.c:17-37 registers the CPU backend, and Metal on
 * request; this registers hip_backend the same way).
 *
 * TEST INFRASTRUCTURE, included by tests/live/engine_live.c and
 * tests/live/py_hip.c. Both are built (oracle/Makefile) from the engine's
 * sources where they lie, with -Dthvm_init=thvm_init_engine: the engine's own
 * thvm_init is compiled under that name, and the includer, after
 * `#undef thvm_init`, gets the engine's entry point back from here with the
 * branch added. The branch is the one written out for maintainers:
 *   - "hip" (or "gpu") as the default device: init the backend; on success
 *     register it as device THVM_DEV_HIP and make it the default, otherwise
 *     print and stay on the CPU (the Metal branch's behaviour,
 *     src/ctx/init.c:32-34);
 *   - thvm_free (src/ctx/init.c:65-77) then shuts it down with every other
 *     registered backend.
 * hip_backend comes from libthvm_hip.so, loaded with dlopen (the engine is
 * not linked against it here) before thvm_init("hip") is called.
 */
#ifndef THVM_TEST_HIP_INIT_H
#define THVM_TEST_HIP_INIT_H

#include <dlfcn.h>

#define THVM_DEV_HIP 2

/* the vtable thvm_init("hip") registers (hip_backend, or a wrapper of it) */
static Backend *g_hip_backend;
/* the library it came from */
static void *g_hip_lib;

/* dlopen()s the backend library and takes its `hip_backend`; 0, or -1 */
static int hip_backend_load(const char *lib_path, int global) {
    g_hip_lib = dlopen(lib_path, RTLD_NOW | (global ? RTLD_GLOBAL : RTLD_LOCAL));
    if (!g_hip_lib) {
        fprintf(stderr, "hip_backend_load: %s\n", dlerror());
        return -1;
    }
    g_hip_backend = (Backend *)dlsym(g_hip_lib, "hip_backend");
    return g_hip_backend ? 0 : -1;
}

TinyHVM *thvm_init_engine(const char *default_device);
TinyHVM *thvm_init(const char *default_device);

TinyHVM *thvm_init(const char *default_device) {
    TinyHVM *ctx = thvm_init_engine(default_device);
    if (ctx && default_device && (strcmp(default_device, "hip") == 0 || strcmp(default_device, "gpu") == 0)) {
        if (g_hip_backend && g_hip_backend->init && g_hip_backend->init() == 0) {
            ctx->backends[THVM_DEV_HIP] = g_hip_backend;
            if (ctx->n_backends < THVM_DEV_HIP + 1) ctx->n_backends = THVM_DEV_HIP + 1;
            ctx->default_device = THVM_DEV_HIP;
        } else {
            fprintf(stderr, "TinyHVM: requested hip backend unavailable; using cpu\n");
        }
    }
    return ctx;
}

#endif
