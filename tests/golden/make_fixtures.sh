#!/bin/sh
# Regenerates the kernel-trace fixtures in this directory from the TinyHVM
# engine (its CPU backend is the reference). Needs the engine sources at
# $REF (default /root/reference/src); builds oracle/_ref/capture first.
#   exec mode (-x): kernels run on the engine's CPU backend; SNAPSHOT records
#                   hold its outputs (the golden vectors).
#   record mode:    kernels are recorded only (full-size workloads); inputs
#                   are generator specs.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
make -s -C "$ROOT/oracle" ref
CAP="$ROOT/oracle/_ref/capture"
cd "$HERE"
# fused elementwise + reduce: sum(relu(a*b+c), -1) and dA = (a*b+c > 0) * b
$CAP fused fused_64x256.trc 64 256
$CAP fused fused_3x1000.trc 3 1000
$CAP fused fused_5x7.trc 5 7
