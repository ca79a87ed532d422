/*
 * noalloc.h - the static device workspace of the no-allocation dispatch
 * (thvm_hip_dispatch_uop_kernel_noalloc). noalloc.hip holds the array; this
 * header is shared by it and the plain-C host code.
 */
#ifndef THVM_NOALLOC_H
#define THVM_NOALLOC_H

#include "thvm_hip.h"

/* bytes of the array on each GPU: THVM_HIP_NOALLOC_SCRATCH_BYTES (thvm_hip.h) */
#define THVM_NOALLOC_MAX_DEVICES 64

#ifdef __cplusplus
extern "C" {
#endif
/* Looks up the array's device address on `device`, which must be the current
 * device; 0 on success, -1 on failure. Once per device. */
int   thvm_noalloc_scratch_init(int device);
/* The address found by thvm_noalloc_scratch_init, or NULL. */
void *thvm_noalloc_scratch_ptr(int device);
#ifdef __cplusplus
}
#endif

#endif
