#!/bin/bash
# Writes tests/golden/vision_view1024.f32: the oracle's features of the timed
# vision configuration (the model's dims, 12 SAM + 24 CLIP layers, the
# xorshift weights of seed 3 and the 1024-pixel image of seed 3 that
# tests/cpp/rocm_vision_test.cpp generates), with and without the device's
# bf16 input rounding: 2 x [256, 1280] fp32, raw. Runs on the host only
# (rocm_vision_test --golden-write needs no device); the GPU test
# (tests/test_gpu_vision_ops.py) regenerates the same weights and compares
# the device encoder with this file.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
root="$(cd "$here/../.." && pwd)"
make -s -C "$root/oracle"
make -s -C "$root/grpc-unlimited-ocr_amd" build/rocm_vision_test 2>/dev/null || make -s -C "$root/grpc-unlimited-ocr_amd"
"$root/grpc-unlimited-ocr_amd/build/rocm_vision_test" --golden-write "$here/vision_view1024.f32"
