/*
 * fake_hip.c - a host-memory stand-in for the few HIP runtime calls the
 * buffer pool (tinyhvm_amd/csrc/pool.c) makes, so the pool's bookkeeping can
 * be tested on a machine without a GPU and under AddressSanitizer: device
 * "memory" is malloc'd, copies are memcpy, streams and events do nothing.
 * hipMalloc fails once the live total would pass fake_hip_limit, which
 * drives the pool's out-of-memory path.
 */
#include <stdlib.h>
#include <string.h>
#include <hip/hip_runtime_api.h>

size_t fake_hip_limit = (size_t)1 << 40;
size_t fake_hip_live = 0;
unsigned long fake_hip_mallocs = 0, fake_hip_frees = 0;

typedef struct { size_t n; } FakeHdr;

hipError_t hipMalloc(void **p, size_t n) {
    if (fake_hip_live + n > fake_hip_limit) {
        *p = NULL;
        return hipErrorOutOfMemory;
    }
    FakeHdr *h = malloc(sizeof(FakeHdr) + 256 + n);
    if (!h) return hipErrorOutOfMemory;
    h->n = n;
    fake_hip_live += n;
    fake_hip_mallocs++;
    *p = (char *)h + 256;   /* 256-byte aligned offset from the header, like device blocks */
    memset(*p, 0xA5, n);
    return hipSuccess;
}

hipError_t hipFree(void *p) {
    if (!p) return hipSuccess;
    FakeHdr *h = (FakeHdr *)((char *)p - 256);
    fake_hip_live -= h->n;
    fake_hip_frees++;
    free(h);
    return hipSuccess;
}

hipError_t hipHostMalloc(void **p, size_t n, unsigned int flags) {
    (void)flags;
    *p = malloc(n);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}

/* host memory stands for device memory here */
hipError_t hipHostGetDevicePointer(void **dev, void *host, unsigned int flags) {
    (void)flags;
    *dev = host;
    return hipSuccess;
}

hipError_t hipHostFree(void *p) {
    free(p);
    return hipSuccess;
}

hipError_t hipMemcpyAsync(void *dst, const void *src, size_t n, hipMemcpyKind kind, hipStream_t s) {
    (void)kind; (void)s;
    memmove(dst, src, n);
    return hipSuccess;
}

hipError_t hipStreamSynchronize(hipStream_t s) { (void)s; return hipSuccess; }
hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned flags) {
    (void)flags;
    *e = (hipEvent_t)malloc(8);
    return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t e) { free((void *)e); return hipSuccess; }
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s) { (void)e; (void)s; return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t e) { (void)e; return hipSuccess; }
hipError_t hipGetLastError(void) { return hipSuccess; }
const char *hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "fake error"; }
