"""Pins the vision half of the CPU oracle (oracle/uocr_oracle_vision.c)
before any GPU result is judged against it:

* bit equality with the reference's own ops (src/backend/reference/ops.cpp)
  through the committed golden vectors (tests/golden/vision_vectors.npz,
  written by tests/golden/make_vision_golden.py over oracle/_ref) and, where
  oracle/_ref was built, on further random shapes;
* independent forms: a direct fp64 convolution loop (not im2col), numpy's
  transposes, torch's antialiased bicubic and linear interpolation (the
  filters the reference restates), an fp64 softmax attention, and an fp64
  brute force of SAM's decomposed relative-position bias;
* the reference's own layout checks of the encoder (tests/vision_test.cpp:
  token counts, the separator last, a newline after every global grid row)
  and residual identities (a block whose output projections are zero leaves
  the stream as it was);
* a planted slip (kernel axes swapped in a numpy im2col) that the direct
  convolution check rejects.
"""

import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "vision_vectors.npz")


def rng(seed=0):
    return np.random.default_rng(seed)


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def conv_direct(x, w, b, stride, pad):
    """fp64 convolution by its definition (no im2col)."""
    x, w = x.astype(np.float64), w.astype(np.float64)
    c, h, wd = x.shape
    o, _, kh, kw = w.shape
    oh, ow = (h + 2 * pad - kh) // stride + 1, (wd + 2 * pad - kw) // stride + 1
    xp = np.zeros((c, h + 2 * pad, wd + 2 * pad))
    xp[:, pad:pad + h, pad:pad + wd] = x
    out = np.zeros((o, oh, ow))
    for oy in range(oh):
        for ox in range(ow):
            win = xp[:, oy * stride:oy * stride + kh, ox * stride:ox * stride + kw]
            out[:, oy, ox] = np.tensordot(w, win, axes=([1, 2, 3], [0, 1, 2]))
    if b is not None:
        out += np.asarray(b, np.float64)[:, None, None]
    return out


# ---- against the reference's own code -------------------------------------------------------


def test_conv2d_bit_equals_reference_golden(orc, gold):
    for tag in ("patch", "conv3"):
        stride, pad = gold[f"conv_{tag}_shape"]
        b = gold[f"conv_{tag}_b"] if f"conv_{tag}_b" in gold else None
        got = orc.conv2d(gold[f"conv_{tag}_x"], gold[f"conv_{tag}_w"], b, int(stride), int(pad))
        assert same_bits(got, gold[f"conv_{tag}_y"]), tag


def test_channel_norm_attention_and_resizes_bit_equal_reference_golden(orc, gold):
    assert same_bits(orc.layer_norm_channels(gold["lnc_x"], gold["lnc_w"], gold["lnc_b"], 1e-6), gold["lnc_y"])
    got = orc.attention_head(gold["att_q"], gold["att_k"], gold["att_v"], gold["att_bias"], np.float32(0.35))
    assert same_bits(got, gold["att_out"])
    for tag in ("shrink", "grow"):
        y = gold[f"bicubic_{tag}_y"]
        assert same_bits(orc.resize_bicubic_aa(gold[f"bicubic_{tag}_x"], y.shape[1], y.shape[2]), y), tag
        y = gold[f"linrows_{tag}_y"]
        assert same_bits(orc.resize_linear_rows(gold[f"linrows_{tag}_x"], y.shape[0]), y), tag


@pytest.fixture(scope="module")
def ref(orc):
    r = orc.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return r


def _p(a):
    return None if a is None else a.ctypes.data


def test_oracle_bit_equals_reference_vision_ops(orc, ref):
    g = rng(30)
    for c, h, w, o, k, stride, pad in [(3, 64, 64, 8, 16, 16, 0), (6, 8, 8, 5, 3, 1, 1), (4, 7, 7, 3, 3, 2, 1),
                                       (12, 4, 4, 16, 3, 2, 1), (9, 5, 5, 2, 1, 1, 0)]:
        x = g.standard_normal((c, h, w), dtype=np.float32)
        wt = (0.3 * g.standard_normal((o, c, k, k))).astype(np.float32)
        b = g.standard_normal(o, dtype=np.float32)
        oh, ow = orc.conv_out(h, k, stride, pad), orc.conv_out(w, k, stride, pad)
        want = np.empty((o, oh, ow), np.float32)
        ref.ref_conv2d(_p(x), c, h, w, _p(wt), _p(b), o, k, k, stride, pad, _p(want))
        assert same_bits(orc.conv2d(x, wt, b, stride, pad), want), (c, h, w, o, k, stride, pad)
    for c, h, w, oh, ow in [(24, 64, 64, 8, 8), (16, 16, 16, 2, 2), (5, 64, 64, 40, 40), (3, 16, 16, 16, 16),
                            (2, 5, 3, 11, 13)]:
        x = g.standard_normal((c, h, w), dtype=np.float32)
        want = np.empty((c, oh, ow), np.float32)
        ref.ref_resize_bicubic_aa(_p(x), c, h, w, oh, ow, _p(want))
        assert same_bits(orc.resize_bicubic_aa(x, oh, ow), want), (c, h, w, oh, ow)
        hwc = np.empty((h, w, c), np.float32)
        ref.ref_chw_to_hwc(_p(x), c, h, w, _p(hwc))
        assert same_bits(orc.chw_to_hwc(x), hwc)
        back = np.empty((c, h, w), np.float32)
        ref.ref_hwc_to_chw(_p(hwc), h, w, c, _p(back))
        assert same_bits(orc.hwc_to_chw(hwc), back)
    for n, d, m in [(127, 12, 15), (27, 12, 27), (127, 64, 79), (5, 3, 1)]:
        x = g.standard_normal((n, d), dtype=np.float32)
        want = np.empty((m, d), np.float32)
        ref.ref_resize_linear_rows(_p(x), n, d, m, _p(want))
        assert same_bits(orc.resize_linear_rows(x, m), want), (n, d, m)
    for lq, lk, d, dv, with_bias in [(196, 196, 12, 12, True), (5, 257, 8, 8, False), (3, 4, 16, 5, True)]:
        q, k = g.standard_normal((lq, d), dtype=np.float32), g.standard_normal((lk, d), dtype=np.float32)
        v = g.standard_normal((lk, dv), dtype=np.float32)
        bias = g.standard_normal((lq, lk), dtype=np.float32) if with_bias else None
        want = np.empty((lq, dv), np.float32)
        ref.ref_attention_head(_p(q), lq, _p(k), lk, d, _p(v), dv, _p(bias), np.float32(0.25), _p(want))
        assert same_bits(orc.attention_head(q, k, v, bias, np.float32(0.25)), want)


# ---- independent forms ----------------------------------------------------------------------


@pytest.mark.parametrize("c,h,w,o,k,stride,pad", [(3, 32, 32, 4, 16, 16, 0), (5, 9, 9, 4, 3, 1, 1),
                                                  (4, 8, 8, 6, 3, 2, 1), (7, 5, 5, 3, 1, 1, 0)])
def test_conv2d_is_the_direct_convolution(orc, c, h, w, o, k, stride, pad):
    g = rng(31 + c)
    x = g.standard_normal((c, h, w), dtype=np.float32)
    wt = (0.3 * g.standard_normal((o, c, k, k))).astype(np.float32)
    b = g.standard_normal(o, dtype=np.float32)
    want = conv_direct(x, wt, b, stride, pad)
    got = orc.conv2d(x, wt, b, stride, pad)
    assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))
    # im2col is the patch matrix whose product with the flattened weight is the convolution
    cols = orc.im2col(x, k, k, stride, pad)
    prod = cols.astype(np.float64) @ wt.reshape(o, -1).T.astype(np.float64) + b
    assert np.allclose(prod.T.reshape(want.shape), want, rtol=0, atol=1e-9 * max(1.0, np.max(np.abs(want))) + 1e-9)


def test_a_swapped_kernel_axis_is_caught_by_the_direct_convolution():
    """A planted slip: an im2col that walks kx before ky."""
    g = rng(32)
    c, h, w, o, k = 3, 6, 6, 2, 3
    x = g.standard_normal((c, h, w), dtype=np.float32)
    wt = g.standard_normal((o, c, k, k)).astype(np.float32)
    xp = np.zeros((c, h + 2, w + 2), np.float32)
    xp[:, 1:-1, 1:-1] = x
    rows = []
    for oy in range(h):
        for ox in range(w):
            rows.append(xp[:, oy:oy + k, ox:ox + k].transpose(0, 2, 1).reshape(-1))  # the slip
    bad = (np.array(rows) @ wt.reshape(o, -1).T).T.reshape(o, h, w)
    assert np.max(np.abs(bad - conv_direct(x, wt, None, 1, 1))) > 1e-3


def test_layout_ops(orc):
    g = rng(33)
    x = g.standard_normal((5, 3, 4), dtype=np.float32)
    assert np.array_equal(orc.chw_to_hwc(x), x.transpose(1, 2, 0))
    assert np.array_equal(orc.hwc_to_chw(orc.chw_to_hwc(x)), x)
    a, b = g.standard_normal((7, 3), dtype=np.float32), g.standard_normal((7, 5), dtype=np.float32)
    assert np.array_equal(orc.concat_cols(a, b), np.concatenate([a, b], axis=1))


def test_channel_layer_norm_is_the_row_norm_over_channels(orc):
    g = rng(34)
    x = 2 * g.standard_normal((6, 4, 5), dtype=np.float32) + 1
    w, b = (1 + 0.1 * g.standard_normal(6)).astype(np.float32), (0.1 * g.standard_normal(6)).astype(np.float32)
    got = orc.layer_norm_channels(x, w, b, 1e-6)
    x64 = x.astype(np.float64)
    mean, var = x64.mean(axis=0), x64.var(axis=0)
    want = (x64 - mean) / np.sqrt(var + 1e-6) * w[:, None, None] + b[:, None, None]
    assert np.max(np.abs(got - want)) < 1e-5


def test_bicubic_resize_is_torchs_antialiased_bicubic(orc):
    torch = pytest.importorskip("torch")
    g = rng(35)
    for c, h, w, oh, ow in [(4, 64, 64, 8, 8), (3, 16, 16, 2, 2), (2, 64, 64, 40, 40), (2, 5, 7, 9, 12)]:
        x = g.standard_normal((c, h, w), dtype=np.float32)
        want = torch.nn.functional.interpolate(torch.from_numpy(x)[None].double(), size=(oh, ow), mode="bicubic",
                                               align_corners=False, antialias=True)[0].numpy()
        got = orc.resize_bicubic_aa(x, oh, ow)
        assert np.max(np.abs(got - want)) < 2e-5 * max(1.0, np.max(np.abs(want))), (c, h, w, oh, ow)
    x = g.standard_normal((2, 9, 9), dtype=np.float32)
    assert np.array_equal(orc.resize_bicubic_aa(x, 9, 9), x)  # same size: the identity
    flat = np.full((1, 64, 64), 0.75, np.float32)
    assert np.max(np.abs(orc.resize_bicubic_aa(flat, 8, 8) - 0.75)) < 1e-6  # normalised taps


def test_linear_row_resize_is_torchs_linear_interpolation(orc):
    torch = pytest.importorskip("torch")
    g = rng(36)
    for n, d, m in [(127, 12, 15), (27, 4, 53), (9, 3, 9)]:
        x = g.standard_normal((n, d), dtype=np.float32)
        want = torch.nn.functional.interpolate(torch.from_numpy(x.T.copy())[None].double(), size=m, mode="linear",
                                               align_corners=False)[0].numpy().T
        # the reference forms the source coordinate in fp32 (about 1e-5 off at
        # row 64), torch in fp64: the bar is that coordinate error
        assert np.max(np.abs(orc.resize_linear_rows(x, m) - want)) < 1e-4
    x = g.standard_normal((5, 2), dtype=np.float32)
    assert np.array_equal(orc.resize_linear_rows(x, 5), x)


def test_relative_positions_index_the_table(orc):
    g = rng(37)
    t = g.standard_normal((27, 6), dtype=np.float32)
    got = orc.relative_positions(t, 14)
    for q in range(14):
        for k in range(14):
            assert np.array_equal(got[q, k], t[q - k + 13])
    t = g.standard_normal((127, 6), dtype=np.float32)
    r = orc.resize_linear_rows(t, 15)
    got = orc.relative_positions(t, 8)
    assert all(np.array_equal(got[q, k], r[q - k + 7]) for q in range(8) for k in range(8))


def test_rel_pos_bias_is_the_decomposed_dot_products(orc):
    g = rng(38)
    h, w, d, ldq = 5, 7, 12, 40
    q = g.standard_normal((h * w, ldq), dtype=np.float32)
    rh, rw = g.standard_normal((h, h, d), dtype=np.float32), g.standard_normal((w, w, d), dtype=np.float32)
    got = orc.rel_pos_bias(q, h, w, rh, rw)
    q64 = q[:, :d].astype(np.float64)
    want = np.empty((h * w, h * w))
    for t in range(h * w):
        qy, qx = divmod(t, w)
        by = rh[qy].astype(np.float64) @ q64[t]
        bx = rw[qx].astype(np.float64) @ q64[t]
        want[t] = (by[:, None] + bx[None, :]).reshape(-1)
    assert np.max(np.abs(got - want)) < 1e-5 * np.max(np.abs(want))


def test_attention_head_is_the_softmax_attention(orc):
    g = rng(39)
    q, k, v = (g.standard_normal((9, 8), dtype=np.float32), g.standard_normal((12, 8), dtype=np.float32),
               g.standard_normal((12, 6), dtype=np.float32))
    bias = g.standard_normal((9, 12), dtype=np.float32)
    s = q.astype(np.float64) @ k.T.astype(np.float64) * 0.3 + bias
    p = np.exp(s - s.max(axis=1, keepdims=True))
    want = (p / p.sum(axis=1, keepdims=True)) @ v.astype(np.float64)
    assert np.max(np.abs(orc.attention_head(q, k, v, bias, 0.3) - want)) < 1e-5
    dead = np.full((9, 12), -np.inf, np.float32)
    assert np.array_equal(orc.attention_head(q, k, v, dead, 0.3), np.zeros((9, 6), np.float32))


# ---- the encoder ----------------------------------------------------------------------------


def image(size, seed):
    return rng(seed).uniform(-1, 1, (3, size, size)).astype(np.float32)


@pytest.fixture(scope="module")
def tiny(orc):
    w = orc.tiny_vision_weights()
    return w, orc.VisionModel(w, orc.TINY_SAM, orc.TINY_CLIP, orc.TINY_HIDDEN)


def test_encoder_token_layout(orc, tiny):
    """tests/vision_test.cpp:63-88 on the same tiny model."""
    w, m = tiny
    assert m.encode_view(image(128, 1)).shape == (4, 20)
    base = m.encode_page(image(128, 2))
    assert base.shape[0] == orc.page_image_tokens(2, 2, 1, 1, False) == 2 * 3 + 1
    tiled = m.encode_page(image(128, 3), [image(128, 4), image(128, 5)], 2, 1)
    assert tiled.shape[0] == orc.page_image_tokens(2, 2, 2, 1, True)
    assert np.array_equal(base[-1], w["model.view_seperator"])
    assert np.array_equal(base[2], w["model.image_newline"]) and np.array_equal(base[5], w["model.image_newline"])
    # tiled: two stitched rows of 2 x 2 cells plus a newline, then the global view
    for r in (4, 9, 12, 15):
        assert np.array_equal(tiled[r], w["model.image_newline"])
    assert np.isfinite(tiled).all()
    # the global view's rows are encode_view's rows
    view = m.encode_view(image(128, 3))
    assert np.array_equal(tiled[10:12], view[0:2]) and np.array_equal(tiled[13:15], view[2:4])
    # each tile's cells sit in its columns of the stitched grid
    t0, t1 = m.encode_view(image(128, 4)), m.encode_view(image(128, 5))
    assert np.array_equal(tiled[0:2], t0[0:2]) and np.array_equal(tiled[2:4], t1[0:2])
    assert np.array_equal(tiled[5:7], t0[2:4]) and np.array_equal(tiled[7:9], t1[2:4])


def test_zero_sublayer_outputs_leave_the_stream(orc, tiny):
    """With every block's and layer's output projections (and biases) zero,
    SAM's blocks and CLIP's layers add nothing: the features equal those of
    a model with no blocks and no layers."""
    w, _ = tiny
    z = dict(w)
    for name in list(z):
        if any(s in name for s in ("attn.proj.", "mlp.lin2.", "self_attn.out_proj.", "mlp.fc2.")):
            z[name] = np.zeros_like(z[name])
    deep = orc.VisionModel(z, orc.TINY_SAM, orc.TINY_CLIP, orc.TINY_HIDDEN)
    shallow = orc.VisionModel(z, dict(orc.TINY_SAM, layers=0), dict(orc.TINY_CLIP, layers=0), orc.TINY_HIDDEN)
    img = image(128, 6)
    assert np.array_equal(deep.encode_view(img), shallow.encode_view(img))
    # and a live block does change them
    live = orc.VisionModel(w, orc.TINY_SAM, orc.TINY_CLIP, orc.TINY_HIDDEN)
    assert not np.array_equal(live.encode_view(img), shallow.encode_view(img))


def test_device_rounding_stays_within_the_references_bf16_bar(orc, tiny):
    """The device linear rounds its inputs to bf16; the reference holds its
    device encoder to 2e-2 of the CPU one (tests/cuda_vision_test.cpp:122)."""
    _, m = tiny
    img = image(128, 8)
    a, b = m.encode_page(img, round_x=False), m.encode_page(img, round_x=True)
    err = np.max(np.abs(a - b)) / np.max(np.abs(a))
    assert 0 < err < 2e-2


def test_structural_slips_exceed_the_encoder_bar(orc):
    """The encoder's device bars (1e-2 of the rounded oracle, 2e-2 of the CPU
    arithmetic, at the largest feature) have teeth: on the real widths (2 + 2
    layers, a 256-pixel view) dropping the relative-position tables, making
    the windowed block global, or skipping a CLIP layer each move the
    features by more than 3e-2."""
    sam = dict(image=1024, patch=16, width=768, layers=2, heads=12, mlp=3072, window=14, global_layers=(1,),
               neck=256, net2=512, net3=1024)
    clip = dict(width=1024, layers=2, heads=16, mlp=4096, positions=257)
    g = rng(40)
    w = {}
    for name, shape in orc.vision_tensor_shapes(sam, clip, 1280).items():
        fan = int(np.prod(shape[1:])) if len(shape) in (2, 4) else 1
        scale = min(0.05, 1 / np.sqrt(fan)) if len(shape) in (2, 4) and "pos" not in name else 0.05
        v = (scale * g.standard_normal(shape)).astype(np.float32)
        w[name] = orc.bf16_round(v + 1 if "norm" in name and name.endswith(".weight") else v)
    img = image(256, 41)
    base = orc.VisionModel(w, sam, clip, 1280).encode_view(img)

    def moved(weights, s=sam, c=clip):
        got = orc.VisionModel(weights, s, c, 1280).encode_view(img)
        return np.max(np.abs(got - base)) / np.max(np.abs(base))

    no_rel = {k: (np.zeros_like(v) if "rel_pos" in k else v) for k, v in w.items()}
    assert moved(no_rel) > 3e-2
    assert moved(w, s=dict(sam, global_layers=(0, 1))) > 3e-2
    assert moved(w, c=dict(clip, layers=1)) > 3e-2
