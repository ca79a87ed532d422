#!/bin/sh
# Regenerates the kernel-trace fixtures in this directory from the TinyHVM
# engine, whose CPU backend is the reference. Needs the engine sources at
# $REF (default /root/reference/src); builds oracle/_ref/capture first.
# Exec mode: kernels run on the engine's CPU backend and each dispatch is
# followed by a SNAPSHOT of its output (the golden vectors). Dispatches whose
# masked loads fall outside their buffer (zero padding) are run by the engine
# with its leaves in zero-filled guard memory and marked so (source 2).
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
make -s -C "$ROOT/oracle" ref
CAP="$ROOT/oracle/_ref/capture"
cd "$HERE"
rm -f ./*.trc
# fused elementwise + reduce: y = sum(relu(a*b+c), -1), dA = (a*b+c > 0) * b
$CAP fused fused_64x256.trc 64 256
$CAP fused fused_3x1000.trc 3 1000
$CAP fused fused_5x7.trc 5 7
# dense matmul + bias + relu, backward dX and dW (K >= 256 takes the group reduce)
$CAP linear linear_8x16x12.trc 8 16 12
$CAP linear linear_33x300x40.trc 33 300 40
# 2-layer MLP forward + backward at the benchmark's own size
$CAP mlp mlp_64x784x128x10.trc 64 784 128 10
# LeNet-5 training step (forward, backward, SGD through ASSIGN)
$CAP lenet lenet_b2.trc 2 1
# conv3x3 + batchnorm(train) + relu + maxpool block, forward + backward
$CAP convblock convblock_2x4x8.trc 2 4 8
# the same at 28x28 (image rows not a multiple of the GEMM stage depth)
$CAP convblock convblock_2x4x28.trc 2 4 28
# 64 channels at 8x8 (the convolution's weights fill a 64-wide GEMM tile: operand packing)
$CAP convblock convblock_1x64x8.trc 1 64 8
# max-pool routing at tied maxima (integer-valued activations, positive ties)
$CAP pooltie pooltie_2x4x16.trc 2 4 16
# storage dtypes and casts
$CAP dtypes dtypes.trc
# ASSIGN from strided views (the contiguify slot)
$CAP assign assign.trc
# the legacy per-op slots (op_unary / op_binary / op_mm / op_reduce)
$CAP legacy legacy.trc
# the adam_step slot against the engine's lazy Adam (src/nn/adam.c)
$CAP adam adam.trc
# the engine's own known-answer tests, restated
$CAP known known.trc
# few outputs over long axes (split group reductions)
$CAP longreduce longreduce_4x20000.trc 4 20000
# the engine's FusedOp fallback path (lowering disabled)
THVM_NO_LOWER=1 $CAP fused rs_fused_16x300.trc 16 300
THVM_NO_LOWER=1 $CAP linear rs_linear_8x16x12.trc 8 16 12
THVM_NO_LOWER=1 $CAP dtypes rs_dtypes.trc
THVM_NO_LOWER=1 $CAP convblock rs_convblock_2x4x8.trc 2 4 8
