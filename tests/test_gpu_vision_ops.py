"""GPU parity for the vision encoder's ops (csrc/vision.hip) through the C
ABI, against the oracle (oracle/uocr_oracle_vision.c):

  * im2col, chw_to_hwc, hwc_to_chw, concat_cols, split_heads and
    merge_heads are data movement:
    bit-exact, over the encoder's shapes (the 16 x 16 patch embedding, the
    padded stride-1 and stride-2 3 x 3 convolutions) and ragged ones;
  * rel_pos_bias at 1e-5 of the largest |bias| (fp32 dot products, fused
    multiply-adds on the device);
  * the whole encoder (src/model/rocm/vision.cpp) against the oracle's
    encoder through the plain-main tests/cpp/rocm_vision_test.cpp;
  * rel_pos_softmax_rows against the oracle's rel_pos_bias + add +
    softmax_rows per window at 1e-5, over windowed (14 x 14 tokens, several
    windows) and global (32 x 32, 64 x 64 and 72 x 72 tokens: the register
    and the three-pass paths) shapes; a row of -inf scores becomes zeros.
"""

import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from parity import assert_f32_close, dev_f32, host_f32, normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def device(backend):
    if not torch.cuda.is_available() or backend.device_count() == 0:
        pytest.skip("no HIP device")
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


@pytest.mark.parametrize("c,h,w,k,stride,pad", [(3, 64, 64, 16, 16, 0), (8, 16, 16, 3, 1, 1), (8, 16, 16, 3, 2, 1),
                                                (12, 8, 8, 3, 2, 1), (5, 7, 9, 3, 2, 1), (24, 8, 8, 1, 1, 0),
                                                (3, 1024, 1024, 16, 16, 0)])
def test_im2col_is_exact(backend, c, h, w, k, stride, pad):
    x = normal(600 + c, (c, h, w))
    want = oracle.im2col(x, k, k, stride, pad)
    cols = torch.full(want.shape, float("nan"), device="cuda")
    backend.im2col(dev_f32(x), k, k, stride, pad, cols)
    assert np.array_equal(host_f32(cols).view(np.uint32), want.view(np.uint32))
    # into bf16 (the patches with the convolution's rounding): the oracle's
    # patches rounded to bf16, bit for bit
    cols16 = torch.full(want.shape, float("nan"), dtype=torch.bfloat16, device="cuda")
    backend.im2col(dev_f32(x), k, k, stride, pad, cols16)
    assert np.array_equal(cols16.view(torch.int16).cpu().numpy().view(np.uint16), oracle.f32_to_bf16(want))


@pytest.mark.parametrize("c,h,w", [(768, 64, 64), (3, 5, 7), (1024, 16, 16), (65, 3, 67)])
def test_layout_transposes_are_exact(backend, c, h, w):
    x = normal(610 + c, (c, h, w))
    hwc = torch.empty(h, w, c, device="cuda")
    backend.chw_to_hwc(dev_f32(x), hwc)
    assert np.array_equal(host_f32(hwc), oracle.chw_to_hwc(x))
    back = torch.empty(c, h, w, device="cuda")
    backend.hwc_to_chw(hwc, back)
    assert np.array_equal(host_f32(back), x)


def test_concat_cols_is_exact(backend):
    a, b = normal(620, (256, 1024)), normal(621, (256, 1024))
    out = torch.empty(256, 2048, device="cuda")
    backend.concat_cols(dev_f32(a), dev_f32(b), out)
    assert np.array_equal(host_f32(out), oracle.concat_cols(a, b))
    a, b = normal(622, (5, 3)), normal(623, (5, 13))
    out = torch.empty(5, 16, device="cuda")
    backend.concat_cols(dev_f32(a), dev_f32(b), out)
    assert np.array_equal(host_f32(out), oracle.concat_cols(a, b))


@pytest.mark.parametrize("h,w,d,ldq", [(14, 14, 64, 3 * 768), (8, 8, 12, 72), (5, 7, 16, 16), (64, 64, 64, 2304)])
def test_rel_pos_bias(backend, h, w, d, ldq):
    q = normal(630 + h, (h * w, ldq))
    rh, rw = normal(631, (h, h, d)), normal(632, (w, w, d))
    want = oracle.rel_pos_bias(q, h, w, rh, rw)
    bias = torch.full((h * w, h * w), float("nan"), device="cuda")
    backend.rel_pos_bias(dev_f32(q), ldq, h, w, d, dev_f32(rh), dev_f32(rw), bias)
    assert_f32_close(host_f32(bias), want, 1e-5, f"rel_pos_bias {h}x{w} d={d}")


@pytest.mark.parametrize("windows,h,w,d,heads", [(3, 14, 14, 64, 2), (25, 14, 14, 64, 1), (1, 8, 8, 12, 2),
                                                 (1, 32, 32, 64, 1), (1, 64, 64, 64, 1), (1, 72, 72, 16, 1),
                                                 (2, 5, 7, 8, 3)])
def test_rel_pos_softmax_rows(backend, windows, h, w, d, heads):
    """Scores of one head of every window (rows window-major, q rows of
    [q | k | v] per head as the encoder lays them out) against the oracle's
    bias, add and row softmax per window."""
    n, width = h * w, heads * d
    ldq = 3 * width
    head = heads - 1
    q_all = normal(640 + n, (windows * n, ldq))
    scores = normal(641 + n, (windows, n, n)) * 3
    rh, rw = normal(642, (h, h, d)), normal(643, (w, w, d))
    want = np.empty_like(scores)
    for win in range(windows):
        qw = q_all[win * n:(win + 1) * n, head * d:(head + 1) * d]
        b = oracle.rel_pos_bias(qw, h, w, rh, rw)
        want[win] = oracle.softmax_rows(oracle.add(scores[win], b))
    s = dev_f32(scores)
    q = dev_f32(q_all)
    backend.rel_pos_softmax_rows(s, windows, q, ldq, h, w, d, dev_f32(rh), dev_f32(rw), q_offset=head * d)
    assert_f32_close(host_f32(s), want, 1e-5, f"rel_pos_softmax {windows}x{h}x{w}")


def test_rel_pos_softmax_masked_row_is_zero(backend):
    h = w = 4
    n = h * w
    scores = normal(650, (1, n, n))
    scores[0, 3, :] = -np.inf
    q, rh, rw = normal(651, (n, 8)), normal(652, (h, h, 8)), normal(653, (w, w, 8))
    s = dev_f32(scores)
    backend.rel_pos_softmax_rows(s, 1, dev_f32(q), 8, h, w, 8, dev_f32(rh), dev_f32(rw))
    got = host_f32(s)
    assert np.array_equal(got[0, 3], np.zeros(n, np.float32))
    assert np.allclose(got[0].sum(axis=1)[[0, 1, 2, 4]], 1.0, atol=1e-5)


def test_vision_ops_reject_bad_shapes(backend):
    x = torch.zeros(3, 8, 8, device="cuda")
    cols = torch.zeros(64, 27, device="cuda")
    with pytest.raises(ValueError):
        backend.im2col(x, 9, 9, 1, 0, cols)  # kernel larger than the image
    q = torch.zeros(4, 300, device="cuda")
    b = torch.zeros(4, 4, device="cuda")
    with pytest.raises(ValueError):
        backend.rel_pos_bias(q, 300, 2, 2, 300, q, q, b)  # head dim above 256


def test_cpp_rocm_vision_test(backend):
    """The vision encoder against the oracle's (tiny and real-width models,
    base and tiled pages): the plain-main C++ test."""
    binary = os.path.join(os.path.dirname(backend.LIB_PATH), "rocm_vision_test")
    r = subprocess.run([binary], capture_output=True, text=True, timeout=110)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_full_model_view_against_golden(backend):
    """The timed vision configuration itself (the model's dims: 12 SAM and
    24 CLIP layers, the seeded weights of the bench's timing run, one
    1024-pixel view) against the oracle's features of the same model,
    written on the host by tests/golden/make_vision_view_golden.sh: within
    1e-2 of the oracle with the device's bf16 input rounding and 2e-2 of the
    reference's CPU arithmetic (the reference's bar,
    tests/cuda_vision_test.cpp:121-122), and the median element within 1e-3
    of the rounded oracle."""
    binary = os.path.join(os.path.dirname(backend.LIB_PATH), "rocm_vision_test")
    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vision_view1024.f32")
    r = subprocess.run([binary, "--golden-check", golden], capture_output=True, text=True, timeout=110)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.parametrize("rows,parts,heads,hd", [(4900, 3, 12, 64), (65, 3, 16, 64), (7, 1, 2, 12), (3, 2, 5, 4)])
def test_split_and_merge_heads_are_exact(backend, rows, parts, heads, hd):
    x = normal(660 + rows, (rows, parts * heads * hd))
    y = torch.full((parts, heads, rows, hd), float("nan"), device="cuda")
    backend.split_heads(dev_f32(x), parts, heads, hd, y)
    want = x.reshape(rows, parts, heads, hd).transpose(1, 2, 0, 3)
    assert np.array_equal(host_f32(y), want)
    back = torch.full((rows, heads * hd), float("nan"), device="cuda")
    backend.merge_heads(y[parts - 1].contiguous(), back)
    assert np.array_equal(host_f32(back), x.reshape(rows, parts, heads * hd)[:, parts - 1])


@pytest.mark.parametrize("n,offset", [(4096 * 3072, 0), (257 * 4096, 0), (1000003, 0), (77, 1), (8, 0)])
def test_activation_into_bf16_is_the_fp32_op_then_the_rounding(backend, n, offset):
    """gelu_erf_to_bf16 / quick_gelu_to_bf16 (the MLPs' activation with the
    rounding of their second projection) against the fp32 op in place then
    round_bf16, bit for bit; a ragged n and an unaligned x take the
    element-by-element path. Values span the activations' regimes (x up to
    +-12: the erf tail, sigmoid saturation, zeros)."""
    g = np.random.default_rng(900 + n)
    x = (g.standard_normal(n + offset) * 4).astype(np.float32)
    x[offset:offset + min(n, 4)] = [0.0, -12.0, 12.0, -0.0][:min(n, 4)]
    xd = dev_f32(x)[offset:]
    for quick in (False, True):
        want32 = xd.clone()
        if quick:
            backend.quick_gelu(want32)
        else:
            backend.gelu_erf(want32)
        want = torch.empty(n, dtype=torch.bfloat16, device="cuda")
        backend.round_bf16(want32.contiguous(), want)
        got = torch.full((n,), float("nan"), dtype=torch.bfloat16, device="cuda")
        backend.act_to_bf16(xd, got, quick=quick)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"quick={quick} n={n} offset={offset}"


@pytest.mark.parametrize("rows,cols,offset", [(4096, 768, 0), (257, 1024, 0), (8200, 768, 0), (33, 100, 0), (5, 768, 1),
                                              (3, 16384, 0)])
def test_layer_norm_into_bf16_is_the_norm_then_the_rounding(backend, rows, cols, offset):
    """layer_norm_to_bf16 against layer_norm in place on a copy then
    round_bf16, bit for bit, x left as it was: one-wave rows, 4-wave groups
    past 8192 rows, columns not a multiple of 4 and an unaligned x (element
    by element), rows of 16384 columns spread over 4 waves."""
    g = np.random.default_rng(910 + rows + cols)
    x = (g.standard_normal(rows * cols + offset) * 3 + 0.5).astype(np.float32)
    w = (1 + 0.1 * g.standard_normal(cols)).astype(np.float32)
    b = (0.1 * g.standard_normal(cols)).astype(np.float32)
    xd = dev_f32(x)[offset:].view(rows, cols)
    before = xd.clone()
    ref = xd.clone()
    backend.layer_norm(ref, dev_f32(w), dev_f32(b), 1e-6)
    want = torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda")
    backend.round_bf16(ref, want)
    got = torch.full((rows, cols), float("nan"), dtype=torch.bfloat16, device="cuda")
    backend.layer_norm_to_bf16(xd, dev_f32(w), dev_f32(b), got, 1e-6)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"{rows}x{cols} offset {offset}"
    assert torch.equal(xd, before), "x is read only"


def test_layer_norm_into_bf16_rejects_rows_too_wide(backend):
    x = torch.zeros(1, 16385, device="cuda")
    w = torch.ones(16385, device="cuda")
    y = torch.empty(1, 16385, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        backend.layer_norm_to_bf16(x, w, w, y, 1e-6)


def test_fused_producers_take_empty_inputs_and_refuse_bad_ones(backend):
    """n = 0 / rows = 0 are no-ops; null pointers are refused before any
    launch."""
    x = torch.zeros(0, device="cuda")
    y = torch.zeros(0, dtype=torch.bfloat16, device="cuda")
    backend.act_to_bf16(x, y)
    backend.act_to_bf16(x, y, quick=True)
    w = torch.ones(8, device="cuda")
    backend.layer_norm_to_bf16(torch.zeros(0, 8, device="cuda"), w, w, torch.zeros(0, 8, dtype=torch.bfloat16,
                                                                                    device="cuda"), 1e-6)
    lib = backend.lib()
    assert lib.uocr_rocm_gelu_erf_to_bf16(None, None, None, 4) != 0
    assert lib.uocr_rocm_layer_norm_to_bf16(None, None, None, None, None, 2, 8, 1e-6) != 0
    assert lib.uocr_rocm_linear_bf16x_add_ws(None, None, 2, 8, None, 4, None, None, None, 0) != 0
