#!/bin/bash
# Builds libbl_select.so (HIP kernels + C ABI) in place for gfx950.
# -ffp-contract=off / no denormal flushing: every float operation of the path is one IEEE operation,
# as in the reference's float32 arithmetic. Packed FP32 instructions are disabled.
# The grammar and JSON-Schema compilers (host C++ only) are built with g++ and linked in.
set -e
cd "$(dirname "$0")"
HIPCC=${HIPCC:-/opt/rocm/bin/hipcc}
FLAGS="--offload-arch=gfx950 -O3 -std=c++17 -fPIC -shared -ffp-contract=off -fno-gpu-flush-denormals-to-zero \
 -Xclang -target-feature -Xclang -packed-fp32-ops -Wno-unused-result -Wno-unused-value"
mkdir -p _build
g++ -O2 -std=c++17 -fPIC -c -o _build/bl_grammar.o csrc/bl_grammar.cpp
g++ -O2 -std=c++17 -fPIC -c -o _build/bl_schema.o csrc/bl_schema.cpp
$HIPCC $FLAGS -o libbl_select.so csrc/bl_kernels.hip csrc/bl_api.hip -x none _build/bl_grammar.o _build/bl_schema.o "$@"
