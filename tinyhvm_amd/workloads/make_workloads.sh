#!/bin/sh
# Regenerates the benchmark workload traces in this directory from the TinyHVM
# engine (sources at $REF, default /root/reference/src; builds
# oracle/_ref/capture first). Record-only (-n): the kernels are not run on the
# CPU and the inputs are stored as generator specs, so each trace is small.
#   fused_8192x8192      y = sum(relu(a*b+c), -1) and dA, a/b/c [8192,8192]
#   linear_4096          relu(X @ W + b) and dX, dW at 4096^3
#   linear_8x4096x4096   the same with 8 rows of X (CPU-baseline slice)
#   lenet_b256           one LeNet-5 training step at batch 256
#   lenet_b64            the same at batch 64 (CPU-baseline sample)
#   convblock_b64        conv3x3 64->64 pad 1 + batchnorm + relu + maxpool 2,
#                        forward and backward, x [64,64,56,56]
#   convblock_b1         the same at batch 1 (CPU-baseline sample)
#   mlp_64x784x128x10    2-layer MLP forward + backward at batch 64
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
make -s -C "$ROOT/oracle" ref
CAP="$ROOT/oracle/_ref/capture"
cd "$HERE"
$CAP -n fused fused_8192x8192.trc 8192 8192
$CAP -n linear linear_4096.trc 4096 4096 4096
$CAP -n linear linear_8x4096x4096.trc 8 4096 4096
$CAP -n lenet lenet_b256.trc 256 1
$CAP -n lenet lenet_b64.trc 64 1
$CAP -n convblock convblock_b64.trc 64 64 56
$CAP -n convblock convblock_b1.trc 1 64 56
$CAP -n mlp mlp_64x784x128x10.trc 64 784 128 10
