"""Guards on the gfx950 machine code of the product kernels, read from the
assembly hipcc writes for each source in grpc-unlimited-ocr_amd/csrc:

* no write through the scalar data cache (scalar stores or atomics, its
  write-back or discard): every store is a vector memory instruction;
* no packed fp32 arithmetic (v_pk_add_f32, v_pk_mul_f32, v_pk_fma_f32): the
  build turns the packed-fp32 feature off and the kernels use scalar fp32;
* no private (scratch) memory traffic: register spills or an argument struct
  copied to the stack would add HBM bytes to every wave;
* no device-scope cache maintenance (buffer_wbl2 / buffer_inv, what a
  __threadfence() becomes on gfx950): each writes back and invalidates an
  XCD's L2, and a split-K attention that handed its records over through
  one per workgroup measured 6x slower than a second launch."""

import glob
import os
import re
import subprocess
import tempfile

import pytest

from conftest import PKG_DIR, ROOT

SOURCES = sorted(glob.glob(os.path.join(PKG_DIR, "csrc", "*.hip")))
SCALAR_WRITE = re.compile(r"^\s+s_(store|atomic|buffer_store|buffer_atomic|scratch_store|dcache_wb|dcache_discard)",
                          re.M)
PACKED_FP32 = re.compile(r"^\s+v_pk_(add|mul|fma)_f32", re.M)
SCRATCH = re.compile(r"^\s+scratch_(load|store)", re.M)
L2_FENCE = re.compile(r"^\s+buffer_(wbl2|inv)\b", re.M)


@pytest.mark.parametrize("src", SOURCES, ids=[os.path.basename(s) for s in SOURCES])
def test_kernel_isa(src):
    with tempfile.TemporaryDirectory() as tmp:
        out = os.path.join(tmp, "k.s")
        subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++20", "-O3", "--offload-arch=gfx950", "-Xclang",
                        "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{ROOT}/include", "--cuda-device-only",
                        "-S", "-o", out, src], check=True, capture_output=True)
        asm = open(out).read()
    assert "amdhsa" in asm or ".amdgcn_target" in asm
    assert not SCALAR_WRITE.search(asm), SCALAR_WRITE.search(asm).group(0)
    assert not PACKED_FP32.search(asm), PACKED_FP32.search(asm).group(0)
    assert not SCRATCH.search(asm), SCRATCH.search(asm).group(0)
    assert not L2_FENCE.search(asm), L2_FENCE.search(asm).group(0)
