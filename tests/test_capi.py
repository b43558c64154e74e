"""The C ABI on the CPU: the library loads, exports every entry point that
include/uocr_rocm.h declares, and rejects bad arguments with
UOCR_ROCM_INVALID_ARGUMENT and a "<what>: <detail>" message before touching
a device, which is the reference's std::invalid_argument convention
(src/backend/cuda/decode_ops.cu:239, ops.cu:569,655). No call here reaches
a kernel launch."""

import ctypes
import os
import re
import subprocess

import pytest

from conftest import PKG_DIR, ROOT

HEADER = os.path.join(ROOT, "include", "uocr_rocm.h")


def declared():
    text = open(HEADER).read()
    return re.findall(r"UOCR_ROCM_API\s+[\w\s\*]+?\b(uocr_rocm_\w+)\s*\(", text)


def test_every_declared_symbol_is_exported(backend):
    names = declared()
    assert len(names) == len(set(names)) >= 40
    out = subprocess.run(["nm", "-D", "--defined-only", backend.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (uocr_rocm_\w+)", out))
    assert set(names) <= exported, sorted(set(names) - exported)
    assert set(backend._SIGNATURES) == set(names)


def test_library_loads_with_signatures(backend):
    lib = backend.lib()
    for name in declared():
        assert getattr(lib, name) is not None
    assert lib.uocr_rocm_abi_version() >> 16 == 1
    assert lib.uocr_rocm_status_string(backend.INVALID_ARGUMENT) == b"invalid argument"
    assert isinstance(backend.device_count(), int)


def test_host_library_and_cpp_test_are_built():
    host = os.path.join(PKG_DIR, "build", "libuocr_rocm_host.so")
    ctypes.CDLL(host)  # the C++23 uocr::rocm layer links against the C ABI
    assert os.access(os.path.join(PKG_DIR, "build", "rocm_ops_test"), os.X_OK)


def test_cpp_test_skips_without_device(backend):
    if backend.device_count() != 0:
        pytest.skip("a device is present; the GPU suite runs this binary")
    r = subprocess.run([os.path.join(PKG_DIR, "build", "rocm_ops_test")], capture_output=True, text=True, timeout=60)
    assert r.returncode == 77, r.stderr


def _invalid(backend, name, *args, detail=""):
    lib = backend.lib()
    status = getattr(lib, name)(*args)
    assert status == backend.INVALID_ARGUMENT, (name, status)
    msg = lib.uocr_rocm_last_error().decode()
    assert msg.startswith(name + ":") and detail in msg, msg
    with pytest.raises(ValueError):
        backend.check(status)


FAKE = 0x10000  # an aligned non-null address; never dereferenced: validation fails first


def test_shape_errors(backend):
    _invalid(backend, "uocr_rocm_rms_norm", None, FAKE, FAKE, -1, 64, 1e-6, detail="rows")
    _invalid(backend, "uocr_rocm_rms_norm_bf16", None, FAKE, FAKE, 4, 0, 1e-6, detail="cols")
    _invalid(backend, "uocr_rocm_layer_norm", None, FAKE, FAKE, None, 4, 64, 1e-6, detail="null")
    _invalid(backend, "uocr_rocm_add_rms_norm_bf16", None, FAKE, FAKE, FAKE, FAKE, 4, 64, 1e-6, detail="distinct")
    _invalid(backend, "uocr_rocm_gelu_erf", None, FAKE, -5, detail="n")
    _invalid(backend, "uocr_rocm_silu_mul", None, FAKE, FAKE, 8, detail="distinct")
    _invalid(backend, "uocr_rocm_add_inplace", None, FAKE, FAKE, 8, detail="distinct")
    _invalid(backend, "uocr_rocm_swiglu_bf16", None, FAKE, FAKE + 64, 4, 16, detail="overlap")
    _invalid(backend, "uocr_rocm_swiglu", None, FAKE, FAKE, 4, 0, detail="ffn")


def test_rope_errors(backend):
    args = (None, FAKE, 1, 2)
    _invalid(backend, "uocr_rocm_rope", *args, 7, None, None, FAKE, 3, None, 0, 0, 0, 0, detail="even")
    _invalid(backend, "uocr_rocm_rope", *args, 8, None, None, FAKE, 3, None, 0, 0, 0, 0, detail="dim / 2")
    _invalid(backend, "uocr_rocm_rope", *args, 1024, None, None, FAKE, 512, None, 0, 0, 0, 0, detail="512")
    _invalid(backend, "uocr_rocm_rope_bf16", *args, 16, None, None, FAKE, 7, None, 1, 2, 0, 0, detail="inv_page")
    _invalid(backend, "uocr_rocm_rope_qk_bf16", None, FAKE, 2, FAKE, 2, 1, 16, None, None, FAKE, 8, None, 0, 0, 0,
             0, detail="distinct")
    _invalid(backend, "uocr_rocm_rope_step", None, FAKE, 2, 16, None, FAKE, 8, None, 0, detail="state")
    _invalid(backend, "uocr_rocm_rope_qk_step", None, FAKE, 2, FAKE, 1, 16, FAKE, FAKE, 9, None, 0,
             detail="n_tok")


def test_gather_errors(backend):
    _invalid(backend, "uocr_rocm_gather_row_bf16", None, FAKE, 100, 100, 64, FAKE, detail="outside")
    _invalid(backend, "uocr_rocm_gather_row_bf16", None, FAKE, 100, -1, 64, FAKE, detail="outside")
    _invalid(backend, "uocr_rocm_gather_rows_bf16", None, FAKE, 100, None, 3, 64, FAKE, detail="index")
    _invalid(backend, "uocr_rocm_embed_step", None, FAKE, 100, None, 64, FAKE, detail="state")
    _invalid(backend, "uocr_rocm_gather_rows_bf16_bf16", None, FAKE, 100, FAKE, 3, 0, FAKE, detail="cols")


def test_empty_shapes_are_noops(backend):
    lib = backend.lib()
    assert lib.uocr_rocm_rms_norm(None, None, None, 0, 64, 1e-6) == 0
    assert lib.uocr_rocm_add_rms_norm_bf16(None, None, None, None, None, 0, 64, 1e-6) == 0
    assert lib.uocr_rocm_layer_norm_bf16(None, None, None, None, 0, 0, 1e-6) == 0
    assert lib.uocr_rocm_gelu_erf_bf16(None, None, 0) == 0
    assert lib.uocr_rocm_swiglu_bf16(None, None, None, 0, 0) == 0
    assert lib.uocr_rocm_rope_qk_bf16(None, None, 16, None, 4, 0, 128, None, None, None, 64, None, 0, 0, 0, 0) == 0
    assert lib.uocr_rocm_gather_rows_bf16(None, None, 10, None, 0, 64, None) == 0
    assert lib.uocr_rocm_copy(None, None, None, 0) == 0
    assert lib.uocr_rocm_zero(None, 0, None) == 0
    assert lib.uocr_rocm_memcpy(None, None, 0, backend.D2D, None) == 0


def test_python_layer_rejects_mismatched_tensors(backend):
    torch = pytest.importorskip("torch")
    x = torch.zeros(4, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        backend.add_rms_norm(x, torch.zeros(4, 8), torch.ones(8), x.clone(), 1e-6)
    with pytest.raises(ValueError):
        backend.rms_norm(torch.zeros(4, 8, dtype=torch.float16), torch.ones(8), 1e-6)
    with pytest.raises(ValueError):
        backend.layer_norm(x, torch.ones(8, dtype=torch.bfloat16), torch.zeros(8), 1e-6)


def test_step_op_errors(backend):
    _invalid(backend, "uocr_rocm_router_norm", None, FAKE, FAKE, -1, 64, 1e-6, detail="rows")
    _invalid(backend, "uocr_rocm_router_norm_bf16", None, FAKE, None, 4, 64, 1e-6, detail="null")
    _invalid(backend, "uocr_rocm_quick_gelu", None, FAKE, -5, detail="n")
    _invalid(backend, "uocr_rocm_softmax_rows", None, FAKE, -1, 64, detail="rows")
    _invalid(backend, "uocr_rocm_softmax_rows", None, FAKE, 4, 0, detail="cols")
    _invalid(backend, "uocr_rocm_scale_add_mask", None, FAKE, 1.0, None, -1, 4, 4, detail="shape")
    _invalid(backend, "uocr_rocm_scale_mask_softmax_rows", None, FAKE, 1.0, None, 2, 4, 0, detail="cols")
    _invalid(backend, "uocr_rocm_gemv_bf16", None, FAKE, 20000, FAKE, 4, None, FAKE, detail="12288")
    _invalid(backend, "uocr_rocm_append_step", None, FAKE, FAKE, 64, None, 16, detail="null")
    _invalid(backend, "uocr_rocm_attend_step", None, FAKE, FAKE, FAKE, 2, 300, None, 1.0, FAKE, FAKE, 64, FAKE,
             detail="256")
    _invalid(backend, "uocr_rocm_attend_step", None, FAKE, FAKE, FAKE, 2, 128, None, 1.0, FAKE, FAKE, 0, FAKE,
             detail="capacity")


def test_copy_errors(backend):
    _invalid(backend, "uocr_rocm_copy", None, FAKE, FAKE + 64, -1, detail="n")
    _invalid(backend, "uocr_rocm_copy", None, FAKE, None, 16, detail="null")
    _invalid(backend, "uocr_rocm_copy", None, FAKE, FAKE + 32, 16, detail="overlap")
    _invalid(backend, "uocr_rocm_copy", None, FAKE + 32, FAKE, 16, detail="overlap")
    _invalid(backend, "uocr_rocm_copy", None, FAKE, FAKE + 64, 1 << 60, detail="too large")
    _invalid(backend, "uocr_rocm_gelu_erf", None, FAKE, 1 << 60, detail="too large")
    # the same buffer on both sides is a copy that changes nothing: no launch
    assert backend.lib().uocr_rocm_copy(None, FAKE, FAKE, 16) == 0


def test_fused_step_op_errors(backend):
    rope = (None, FAKE, FAKE, FAKE, FAKE, FAKE)
    _invalid(backend, "uocr_rocm_attend_rope_kv_step", *rope, 2, 7, None, 1.0, FAKE, FAKE, 3, None, 0, FAKE, 64,
             FAKE, detail="even")
    _invalid(backend, "uocr_rocm_attend_rope_kv_step", *rope, 2, 8, None, 1.0, FAKE, FAKE, 5, None, 0, FAKE, 64,
             FAKE, detail="n_tok")
    _invalid(backend, "uocr_rocm_attend_rope_kv_step", *rope, 2, 8, None, 1.0, FAKE, FAKE, 3, None, 0, FAKE, 64,
             FAKE, detail="inv_page")
    _invalid(backend, "uocr_rocm_add_rms_norm_gemv_bf16", None, FAKE, None, None, None, 1e-6, None, 100, FAKE, 4,
             None, FAKE, detail="multiple of 8")
    _invalid(backend, "uocr_rocm_add_rms_norm_gemv_bf16", None, FAKE, None, None, None, 1e-6, None, 4096, FAKE, 4,
             None, FAKE, detail="multiple of 8")
    _invalid(backend, "uocr_rocm_add_rms_norm_gemv_bf16", None, FAKE, None, FAKE, None, 1e-6, None, 128, FAKE, 4,
             None, FAKE, detail="overlap")
    _invalid(backend, "uocr_rocm_add_rms_norm_gemv_bf16", None, FAKE + 4, None, None, None, 1e-6, None, 128, FAKE, 4,
             None, FAKE, detail="aligned")
    _invalid(backend, "uocr_rocm_add_rms_norm_swiglu_gemv_bf16", None, FAKE, None, None, None, 1e-6, None, 128,
             FAKE, None, 4, FAKE, detail="up")
    # the fused router: experts >= 1, and logits never overlapping the row
    _invalid(backend, "uocr_rocm_add_rms_norm_swiglu_router_gemv_bf16", None, FAKE, None, None, None, 1e-6, None,
             128, FAKE, FAKE, 4, 0x30000, 0x40000, 0, 0x50000, detail="experts in [1, 2^20]")
    _invalid(backend, "uocr_rocm_add_rms_norm_swiglu_router_gemv_bf16", None, FAKE, None, None, None, 1e-6, None,
             128, FAKE, FAKE, 4, 0x30000, 0x40000, 64, FAKE + 64, detail="must not overlap")


def test_expert_op_errors(backend):
    x, scratch, out = 0x10000, 0x20000, 0x30000  # distinct, so only the tested rule fails
    _invalid(backend, "uocr_rocm_expert_topk", None, FAKE, 4, 129, 6, FAKE, FAKE, detail="experts must be in [1, 128]")
    _invalid(backend, "uocr_rocm_expert_topk", None, FAKE, 4, 6, 7, FAKE, FAKE, detail="k must be in [1, experts]")
    _invalid(backend, "uocr_rocm_expert_ffn_one", None, x, 128, 64, FAKE, FAKE, FAKE, 16, FAKE, FAKE, 9, None,
             scratch, out, detail="k must be in [1, 8]")
    _invalid(backend, "uocr_rocm_moe_ffn_one", None, x, 128, 64, FAKE, FAKE, FAKE, 6, FAKE, 7, FAKE, FAKE, 0x40000,
             0x50000, 64, scratch, out, detail="k <= experts")
    _invalid(backend, "uocr_rocm_moe_ffn_one", None, x, 128, 64, FAKE, FAKE, FAKE, 200, FAKE, 6, FAKE, FAKE, 0x40000,
             0x50000, 64, scratch, out, detail="experts must be in [1, 128]")


def test_step_op_empty_shapes_and_scratch_size(backend):
    lib = backend.lib()
    assert lib.uocr_rocm_softmax_rows(None, None, 0, 64) == 0
    assert lib.uocr_rocm_scale_add_mask(None, None, 1.0, None, 0, 4, 4) == 0
    assert lib.uocr_rocm_scale_mask_softmax_rows(None, None, 1.0, None, 0, 4, 4) == 0
    assert lib.uocr_rocm_gemv_bf16(None, None, 128, None, 0, None, None) == 0
    assert lib.uocr_rocm_append_step(None, None, None, 0, None, 16) == 0
    assert lib.uocr_rocm_attend_step(None, None, None, None, 0, 128, None, 1.0, None, None, 64, None) == 0
    assert lib.uocr_rocm_add_rms_norm_gemv_bf16(None, None, None, None, None, 1e-6, None, 128, None, 0, None,
                                                None) == 0
    assert lib.uocr_rocm_attend_scratch_floats(0, 128, 100) == 0
    # records only (no per-key scores): heads x splits x (hd + 2), sized for an fp32 cache; 128 splits at 10
    # heads and 8192 positions, 32 at 2048 (no split under 64 KB of key and value rows), 1 for a 7-key cache
    assert lib.uocr_rocm_attend_scratch_floats(10, 128, 8192) == 10 * 128 * 130
    assert lib.uocr_rocm_attend_scratch_floats(10, 128, 2048) == 10 * 32 * 130
    assert lib.uocr_rocm_attend_scratch_floats(32, 64, 1 << 20) == 32 * 64 * 66
    assert lib.uocr_rocm_attend_scratch_floats(1, 64, 7) == 1 * 1 * 66


def test_masked_attention_workspace_sizes(backend):
    """The masked attention paths' workspaces: the tile map (a word per 1024
    keys per 128 query rows, rounded up to 64 floats), then for the split
    path the split key and value tiles (64 hd floats per 32-key tile and
    slice), and the runs' records (hd + 2 floats per row and run) where the
    row blocks leave slots idle. Invalid shapes give 0."""
    fp32 = backend.attention_workspace_floats
    split = backend.attention_masked_workspace_floats
    for f in (fp32, split):
        assert f(0, 64, 64, 128) == 0 and f(1, 0, 64, 128) == 0 and f(1, 64, 0, 128) == 0
        assert f(1, 64, 64, 96) == 0
    # 48 rows over 48 keys: one map word, no runs
    assert fp32(2, 48, 48, 64) == 64
    assert split(2, 48, 48, 64) == 64 + 2 * 2 * 64 * 64
    # 10 heads x 4096 rows and keys at hd 128: 32 row blocks x 4 words of map;
    # the split path cuts a walk into runs of 80 tiles (2 per block), the fp32
    # path (one workgroup per CU) keeps whole walks
    tiles, blocks = 128, 32
    assert fp32(10, 4096, 4096, 128) == blocks * 4 * 1
    assert split(10, 4096, 4096, 128) == blocks * 4 + 10 * tiles * 64 * 128 + 10 * blocks * 2 * 128 * 130
    # few row blocks over many keys: both cut walks into runs
    assert fp32(1, 128, 8192, 64) > 64
