#!/usr/bin/env bash
# Builds sdpa_rocm.so, the TensorFlow-ROCm op library of Sdpa / SdpaGrad for
# MI355X, in this directory.  It replaces the reference's build.sh (nvcc for
# sm_XX plus g++ against a CUDA TensorFlow): the HIP kernels are compiled by
# hipcc for gfx950 into libsdpa_hip.so, the host kernels by g++ into
# libsdpa_cpu.so (the package Makefile), and the op definitions and
# OpKernels here are compiled against the TensorFlow-ROCm headers and linked
# to both libraries.
#
#   tf_op/build.sh                 (PYTHON=python3 ARCH=gfx950 JOBS=8 by default)
#
# Load it with tf.load_op_library(".../tf_op/sdpa_rocm.so"); sdpa.py does.
set -euo pipefail

HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
PKG="$(dirname "$HERE")"
INC="$(dirname "$PKG")/include"
PYTHON="${PYTHON:-python3}"
ARCH="${ARCH:-gfx950}"
ROCM="${ROCM_PATH:-/opt/rocm}"

if ! "$PYTHON" -c "import tensorflow" >/dev/null 2>&1; then
    echo "tf_op/build.sh: TensorFlow is not importable by $PYTHON; install TensorFlow-ROCm first" >&2
    exit 3
fi

make -s -C "$PKG" -j"${JOBS:-8}" ARCH="$ARCH" libsdpa_hip.so libsdpa_cpu.so

read -r -a TF_CFLAGS <<<"$("$PYTHON" -c 'import tensorflow as tf; print(" ".join(tf.sysconfig.get_compile_flags()))')"
read -r -a TF_LFLAGS <<<"$("$PYTHON" -c 'import tensorflow as tf; print(" ".join(tf.sysconfig.get_link_flags()))')"

# Host code only (the device code lives in libsdpa_hip.so): the ROCm build of
# TensorFlow's headers wants the HIP platform and its include path.
g++ -std=c++17 -O2 -fPIC -shared \
    -DTENSORFLOW_USE_ROCM=1 -D__HIP_PLATFORM_AMD__=1 -DEIGEN_USE_HIP \
    "$HERE/sdpa_ops.cc" "$HERE/sdpa_kernels.cc" \
    -I"$INC" -I"$ROCM/include" "${TF_CFLAGS[@]}" \
    -L"$PKG" -lsdpa_hip -lsdpa_cpu -Wl,-rpath,"$PKG" \
    -L"$ROCM/lib" -lamdhip64 "${TF_LFLAGS[@]}" \
    -o "$HERE/sdpa_rocm.so"
echo "built $HERE/sdpa_rocm.so"
