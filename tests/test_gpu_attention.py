"""GPU parity for the one-pass attention (csrc/attention.hip) through the C
ABI, against the oracle's attention_head (the reference's
src/backend/reference/ops.cpp:219-251: dot(q, k) * scale + bias, softmax
with an fp64 total, probabilities times v) slice by slice:

  * no bias, hd 64 and 128, rows and keys not multiples of the 32-key tile
    or the 128-row workgroup, several slices, head-major operands (few rows:
    the keys split over a workgroup's waves);
  * a mask shared by the slices with -inf entries, a causal pattern and a
    row with every key masked (zeros out), rows != keys;
  * strided operands as the decoder's prefill holds them (q, k, v columns of
    [rows, heads * hd] rows, the output into the heads' columns);
  * SAM's relative-position bias over 14 x 14 windows and a 64 x 64 global
    window (and grids whose width is or is not a multiple of 32), against the
    oracle's rel_pos_bias + attention_head;
Tolerance: 1e-5 of the largest |out| (fp32 sums in another order, the
running-max rescale).
"""

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


def reference(q, k, v, scale, bias=None):
    return np.stack([oracle.attention_head(q[s], k[s], v[s], bias, scale) for s in range(q.shape[0])])


@pytest.mark.parametrize("slices,rows,keys,hd", [(1, 1, 1, 64), (3, 31, 33, 64), (2, 257, 257, 64),
                                                 (2, 130, 1000, 128), (1, 1024, 1024, 64), (16, 65, 65, 64),
                                                 (16, 257, 257, 64), (1, 40, 100, 64), (260, 70, 90, 64)])
def test_attention_against_the_oracle(backend, slices, rows, keys, hd):
    """Head dim 64 without a mask and fewer than 256 workgroups of 128 rows
    split the keys over a workgroup's waves (CLIP's 16 x 257; fewer key
    tiles than waves: 40 x 100); 260 slices take the one-wave-per-32-rows
    kernel."""
    q, k, v = normal(700 + rows, (slices, rows, hd)), normal(701 + keys, (slices, keys, hd)), normal(702, (slices, keys, hd))
    scale = float(np.float32(1 / np.sqrt(hd)))
    want = reference(q, k, v, scale)
    out = torch.full((slices, rows, hd), float("nan"), device="cuda")
    backend.attention(dev_f32(q), dev_f32(k), dev_f32(v), out, slices, rows, keys, hd, scale)
    assert_f32_close(host_f32(out), want, 1e-5, f"attention {slices}x{rows}x{keys} hd {hd}")


def test_attention_with_a_mask(backend):
    slices, rows, keys, hd = 3, 100, 300, 128
    q, k, v = normal(710, (slices, rows, hd)), normal(711, (slices, keys, hd)), normal(712, (slices, keys, hd))
    g = np.random.default_rng(713)
    mask = np.where(g.random((rows, keys)) < 0.3, -np.inf, 0.1 * g.standard_normal((rows, keys))).astype(np.float32)
    for t in range(rows):  # causal beyond key 200 + t
        mask[t, 200 + t:] = -np.inf
    mask[7, :] = -np.inf  # every key masked: zeros
    mask[8, :] = -np.inf
    mask[8, 299] = 0.0  # a single live key at the end of the last tile
    scale = 0.088
    want = reference(q, k, v, scale, mask)
    out = torch.full((slices, rows, hd), float("nan"), device="cuda")
    backend.attention(dev_f32(q), dev_f32(k), dev_f32(v), out, slices, rows, keys, hd, scale, mask=dev_f32(mask))
    got = host_f32(out)
    assert np.array_equal(got[:, 7], np.zeros((slices, hd), np.float32))
    assert_f32_close(got, want, 1e-5, "masked attention")


def test_attention_strided_decoder_layout(backend):
    """q, k, v as the decoder's prefill holds them: head h at columns h * hd
    of [rows, heads * hd] rows (q inside a wider projection row), the output
    written into the heads' columns of [rows, heads * hd]."""
    heads, hd, rows = 4, 128, 77
    width = heads * hd
    proj = normal(720, (rows, 5 * width))  # q | ... wider row
    kc, vc = normal(721, (rows, width)), normal(722, (rows, width))
    q = proj[:, :width].reshape(rows, heads, hd).transpose(1, 0, 2)
    k, v = kc.reshape(rows, heads, hd).transpose(1, 0, 2), vc.reshape(rows, heads, hd).transpose(1, 0, 2)
    mask = np.triu(np.full((rows, rows), -np.inf, np.float32), 1)
    want = reference(q, k, v, 0.1, mask).transpose(1, 0, 2).reshape(rows, width)
    out = torch.full((rows, width), float("nan"), device="cuda")
    backend.attention(dev_f32(proj), dev_f32(kc), dev_f32(vc), out, heads, rows, rows, hd, 0.1, mask=dev_f32(mask),
                      strides={"q": (0, 5 * width, hd), "k": (0, width, hd), "v": (0, width, hd),
                               "out": (0, width, hd)})
    assert_f32_close(host_f32(out), want, 1e-5, "strided attention")


@pytest.mark.parametrize("windows,heads,h,w,hd", [(4, 3, 14, 14, 64), (1, 2, 64, 64, 64), (2, 1, 5, 7, 64),
                                                   (2, 1, 5, 32, 64), (1, 2, 3, 64, 64), (1, 1, 6, 32, 128)])
def test_attention_rel_pos_against_the_oracle(backend, windows, heads, h, w, hd):
    """Grid widths of whole 32-key tiles (32, 64) take the per-tile bias
    terms, with h not a multiple of 4 among them; 14 and 7 the per-key
    lookups."""
    n = h * w
    slices = heads * windows
    q, k, v = normal(730 + n, (slices, n, hd)), normal(731 + n, (slices, n, hd)), normal(732, (slices, n, hd))
    rh, rw = normal(733, (h, h, hd)) * 0.3, normal(734, (w, w, hd)) * 0.3
    scale = 0.125
    want = np.stack([oracle.attention_head(q[s], k[s], v[s], oracle.rel_pos_bias(q[s], h, w, rh, rw), scale)
                     for s in range(slices)])
    out = torch.full((slices, n, hd), float("nan"), device="cuda")
    backend.attention_rel_pos(dev_f32(q), dev_f32(k), dev_f32(v), out, slices, h, w, hd, scale, dev_f32(rh),
                              dev_f32(rw))
    assert_f32_close(host_f32(out), want, 1e-5, f"rel-pos attention {windows}x{heads} {h}x{w}")
    # the dots formed beforehand into a workspace (NaN-filled: every entry read is written)
    floats = backend.attention_rel_pos_workspace_floats(slices, h, w)
    assert floats >= slices * n * (h + w)
    ws = torch.full((floats,), float("nan"), device="cuda")
    out2 = torch.full((slices, n, hd), float("nan"), device="cuda")
    backend.attention_rel_pos(dev_f32(q), dev_f32(k), dev_f32(v), out2, slices, h, w, hd, scale, dev_f32(rh),
                              dev_f32(rw), workspace=ws)
    assert_f32_close(host_f32(out2), want, 1e-5, f"rel-pos attention with a dot table {windows}x{heads} {h}x{w}")
    small = torch.zeros(1, device="cuda")  # a workspace too small: the workgroups form their own dots
    out3 = torch.full((slices, n, hd), float("nan"), device="cuda")
    backend.attention_rel_pos(dev_f32(q), dev_f32(k), dev_f32(v), out3, slices, h, w, hd, scale, dev_f32(rh),
                              dev_f32(rw), workspace=small)
    assert torch.equal(out3, out)


def test_attention_rejects_bad_shapes(backend):
    x = torch.zeros(2, 8, 96, device="cuda")
    with pytest.raises(ValueError):
        backend.attention(x, x, x, x, 2, 8, 8, 96, 1.0)  # head dim 96
    y = torch.zeros(1, 8, 64, device="cuda")
    with pytest.raises(ValueError):
        backend.attention_rel_pos(y, y, y, y, 1, 200, 100, 64, 1.0, y, y)  # h + w above 256


@pytest.mark.parametrize("windows,heads,h,w", [(3, 2, 14, 14), (2, 3, 5, 32)])
def test_attention_rel_pos_windows_straight_from_the_rows(backend, windows, heads, h, w):
    """Slice (head, window) read straight from a window-major qkv projection's
    rows and written into the merged rows: against the oracle per (head,
    window) at 1e-5."""
    hd, n = 64, h * w
    width = heads * hd
    qkv = normal(740 + n, (windows * n, 3 * width))
    rh, rw = normal(741, (h, h, hd)) * 0.3, normal(742, (w, w, hd)) * 0.3
    scale = 0.125
    want = np.zeros((windows * n, width), np.float32)
    for win in range(windows):
        rows = qkv[win * n:(win + 1) * n]
        for head in range(heads):
            q = rows[:, head * hd:(head + 1) * hd]
            k = rows[:, width + head * hd:width + (head + 1) * hd]
            v = rows[:, 2 * width + head * hd:2 * width + (head + 1) * hd]
            want[win * n:(win + 1) * n, head * hd:(head + 1) * hd] = oracle.attention_head(
                q, k, v, oracle.rel_pos_bias(q, h, w, rh, rw), scale)
    out = torch.full((windows * n, width), float("nan"), device="cuda")
    ws = torch.full((backend.attention_rel_pos_workspace_floats(heads * windows, h, w),), float("nan"), device="cuda")
    backend.attention_rel_pos_windows(dev_f32(qkv), out, heads, windows, h, w, hd, scale, dev_f32(rh), dev_f32(rw), ws)
    assert_f32_close(host_f32(out), want, 1e-5, f"rel-pos attention over {windows} windows x {heads} heads")


@pytest.mark.parametrize("windows,heads,h,w,amp", [(25, 12, 14, 14, 1.0), (1, 12, 64, 64, 1.0), (3, 2, 7, 9, 1.0),
                                                   (2, 3, 5, 32, 1.0), (3, 2, 1, 32, 1.0), (1, 2, 2, 32, 1.0),
                                                   (1, 2, 8, 32, 6.0), (2, 2, 5, 6, 1.0), (1, 2, 3, 20, 1.0),
                                                   (2, 2, 14, 14, 6.0), (1, 2, 2, 40, 1.0)])
def test_attention_rel_pos_windows_into_bf16_is_the_rounded_output(backend, windows, heads, h, w, amp):
    """The windows' attention written in bf16 (the rounding the output
    projection applies): the fp32 output then round_bf16, SAM's windowed and
    global (one 64 x 64 window) layers. Grids of whole 32-key tile rows, and
    grids under 32 wide (4, 2 or 1 grid rows per key tile: widths 6, 9 and
    14, 20), take the products on the bf16 matrix cores with split operands,
    which moves some outputs across a bf16 rounding boundary: there every
    element is within one bf16 step of the fp32 output, most equal to its
    rounding, and the result within 2^-8 of the oracle (a bf16 step: the
    output's own rounding and a moved boundary). Other widths (40) keep the
    fp32 products: bitwise. One tile, two tiles, an odd count, a last tile
    with grid rows past the grid; amp 6 spreads the scores (standard
    deviation about 36) so that later tiles pass a row's reference point by
    more than the kernel's slack and the sums are rescaled mid-row."""
    hd, n = 64, h * w
    width = heads * hd
    qkv = dev_f32(normal(750 + n, (windows * n, 3 * width)) * np.float32(amp))
    rh, rw = dev_f32(normal(751, (h, h, hd)) * 0.3), dev_f32(normal(752, (w, w, hd)) * 0.3)
    ws = torch.empty(backend.attention_rel_pos_workspace_floats(heads * windows, h, w), device="cuda")
    out = torch.empty(windows * n, width, device="cuda")
    backend.attention_rel_pos_windows(qkv, out, heads, windows, h, w, hd, 0.125, rh, rw, ws)
    want = torch.empty(windows * n, width, dtype=torch.bfloat16, device="cuda")
    backend.round_bf16(out, want)
    got = torch.full((windows * n, width), float("nan"), dtype=torch.bfloat16, device="cuda")
    backend.attention_rel_pos_windows(qkv, got, heads, windows, h, w, hd, 0.125, rh, rw, ws)
    torch.cuda.synchronize()
    if w % 32 != 0 and w > 32:
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        return
    got_f = oracle.bf16_to_f32(got.view(torch.int16).cpu().numpy().view(np.uint16))
    out_f = host_f32(out)
    # one bf16 step of each value (the rounding of a value moved across a
    # boundary), with a floor of 2^-14 of the largest for values near zero;
    # spread scores (amp 6) magnify the split's 2^-16 of each score, so
    # there the bar is the oracle's alone, at 2^-6 (a wrong rescale is off
    # by the whole value)
    bar = 2.0**-8 if amp == 1.0 else 2.0**-6
    if w % 32 == 0:
        # a workspace one float short holds the dot table but not the split
        # key and value tiles of a whole-tile grid: the fp32 products, bitwise
        small = torch.empty(ws.numel() - 1, device="cuda")
        got3 = torch.full((windows * n, width), float("nan"), dtype=torch.bfloat16, device="cuda")
        backend.attention_rel_pos_windows(qkv, got3, heads, windows, h, w, hd, 0.125, rh, rw, small)
        assert torch.equal(got3.view(torch.int16), want.view(torch.int16))
    if amp == 1.0:
        tol = 2.0**-8 * np.abs(out_f) + 2.0**-14 * np.abs(out_f).max()
        assert np.all(np.abs(got_f - out_f) <= tol), float(np.max(np.abs(got_f - out_f) - tol))
        assert np.mean(got.view(torch.int16).cpu().numpy() == want.view(torch.int16).cpu().numpy()) > 0.9
    qkv_h = host_f32(qkv)
    for win in range(windows):
        rows = qkv_h[win * n:(win + 1) * n]
        for head in sorted({0, heads - 1}):  # the first and last heads of each window
            q = rows[:, head * hd:(head + 1) * hd]
            k = rows[:, width + head * hd:width + (head + 1) * hd]
            v = rows[:, 2 * width + head * hd:2 * width + (head + 1) * hd]
            want_o = oracle.attention_head(q, k, v, oracle.rel_pos_bias(q, h, w, host_f32(rh), host_f32(rw)), 0.125)
            assert_f32_close(got_f[win * n:(win + 1) * n, head * hd:(head + 1) * hd], want_o, bar,
                             f"split-bf16 products against the oracle, window {win} head {head}")


@pytest.mark.parametrize("slices,rows,keys,hd,masked", [(16, 257, 257, 64, False), (4, 300, 300, 64, False),
                                                        (3, 100, 130, 128, True)])
def test_attention_into_bf16_is_the_rounded_output(backend, slices, rows, keys, hd, masked):
    """The one-pass attention written in bf16 (CLIP's heads with the keys
    split over the waves, the 128-row tiles, a mask, head dim 128): bitwise
    the fp32 output then round_bf16."""
    q = dev_f32(normal(760 + rows, (slices, rows, hd)))
    k = dev_f32(normal(761 + keys, (slices, keys, hd)))
    v = dev_f32(normal(762, (slices, keys, hd)))
    mask = dev_f32(np.where(normal(763, (rows, keys)) > 1.0, -np.inf, 0.0).astype(np.float32)) if masked else None
    out = torch.empty(slices, rows, hd, device="cuda")
    backend.attention(q, k, v, out, slices, rows, keys, hd, 0.125, mask)
    want = torch.empty(slices, rows, hd, dtype=torch.bfloat16, device="cuda")
    backend.round_bf16(out, want)
    got = torch.full((slices, rows, hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    backend.attention(q, k, v, got, slices, rows, keys, hd, 0.125, mask)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def _routed_mask(rows, keys, seed):
    """A prefill's routed mask: query t at position keys - rows + t attends
    its window (the keys of the last 4 32-key blocks up to its position,
    bias 0) and up to 3 earlier blocks with a bias each; -inf elsewhere and
    past its position."""
    g = np.random.default_rng(seed)
    mask = np.full((rows, keys), -np.inf, np.float32)
    for t in range(rows):
        pos = keys - rows + t
        mask[t, max(0, (pos // 32 - 3) * 32):pos + 1] = 0.0
        earlier = pos // 32 - 3
        if earlier > 0:
            for b in g.choice(earlier, size=min(3, earlier), replace=False):
                mask[t, 32 * b:32 * b + 32] = np.float32(0.5 * g.standard_normal())
    return mask


def _test_mask(kind, rows, keys):
    """random: 30% -inf entries, a causal edge, a row with no live key and a
    row whose one live key ends the last tile; dead: the first 128 rows with
    no live key; causal; routed (_routed_mask)."""
    g = np.random.default_rng(773)
    if kind == "random" or kind == "dead":
        mask = np.where(g.random((rows, keys)) < 0.3, -np.inf, 0.1 * g.standard_normal((rows, keys)))
        mask = mask.astype(np.float32)
        if kind == "dead":
            mask[:128] = -np.inf
        else:
            for t in range(rows):
                mask[t, max(1, keys - rows - 50 + t):] = -np.inf
            mask[0, :] = -np.inf
            if rows > 8:
                mask[8, :] = -np.inf
                mask[8, keys - 1] = 0.0
        return mask
    if kind == "causal":
        return np.triu(np.full((rows, keys), -np.inf, np.float32), 1 + keys - rows)
    return _routed_mask(rows, keys, 774)


@pytest.mark.parametrize("slices,rows,keys,hd,kind", [(3, 100, 300, 128, "random"), (2, 150, 3000, 64, "random"),
                                                      (4, 300, 1100, 128, "routed"), (1, 200, 64, 128, "dead"),
                                                      (2, 257, 257, 64, "causal"), (2, 130, 2500, 128, "causal"),
                                                      (1, 1, 1, 64, "causal")])
def test_attention_with_a_workspace(backend, slices, rows, keys, hd, kind):
    """uocr_rocm_attention_ws / _bf16_ws: the fp32 one-pass attention over a
    mask walking only the tiles its row blocks attend (a first row block
    with no live key: zeros), few row blocks over many keys (1100, 2500,
    3000) cut into runs whose records a merge launch combines: the oracle at
    the fp32 bar, and the bf16 entry bitwise the fp32 one rounded."""
    q, k, v = normal(780 + rows, (slices, rows, hd)), normal(781 + keys, (slices, keys, hd)), normal(782, (slices, keys, hd))
    mask = _test_mask(kind, rows, keys)
    scale = float(np.float32(1 / np.sqrt(hd)))
    qd, kd, vd, md = dev_f32(q), dev_f32(k), dev_f32(v), dev_f32(mask)
    ws = torch.empty(backend.attention_workspace_floats(slices, rows, keys, hd), device="cuda")
    out = torch.full((slices, rows, hd), float("nan"), device="cuda")
    backend.attention(qd, kd, vd, out, slices, rows, keys, hd, scale, md, workspace=ws)
    want16 = torch.empty(slices, rows, hd, dtype=torch.bfloat16, device="cuda")
    backend.round_bf16(out, want16)
    got16 = torch.full((slices, rows, hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    backend.attention(qd, kd, vd, got16, slices, rows, keys, hd, scale, md, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(got16.view(torch.int16), want16.view(torch.int16))
    got = host_f32(out)
    dead = ~np.isfinite(mask).any(axis=1)
    assert np.array_equal(got[:, dead], np.zeros_like(got[:, dead]))
    assert_f32_close(got, reference(q, k, v, scale, mask), 1e-5, f"attention with a workspace, {kind} mask")
    with pytest.raises(ValueError):  # a workspace one float short
        backend.attention(qd, kd, vd, out, slices, rows, keys, hd, scale, md, workspace=ws[:-1])


@pytest.mark.parametrize("slices,rows,keys,hd,kind,amp", [(3, 100, 300, 128, "random", 1.0),
                                                          (2, 257, 257, 64, "causal", 1.0),
                                                          (4, 300, 1100, 128, "routed", 1.0),
                                                          (1, 1, 33, 128, "random", 1.0),
                                                          (2, 130, 40, 64, "causal", 1.0),
                                                          (2, 200, 2100, 128, "routed", 4.0),
                                                          (1, 200, 64, 128, "dead", 1.0),
                                                          (2, 150, 3000, 64, "random", 1.0),
                                                          (1, 1, 1, 128, "causal", 1.0)])
def test_attention_masked_split_operands(backend, slices, rows, keys, hd, kind, amp):
    """uocr_rocm_attention_masked_bf16_ws: the masked attention into bf16 on
    the bf16 matrix cores with split operands, the workgroups walking only
    the 32-key tiles their 128 rows attend. Masks: random -inf entries with
    a causal edge, a row with no live key and a row whose one live key ends
    the last tile; causal; a prefill's routed mask (window plus selected
    blocks, past the position -inf); a first row block with no live key at
    all (zeros). Few row blocks over many keys (1100, 2100, 3000) cut a
    block's walk into runs of at least 32 live tiles whose partial records
    a merge launch combines. As for SAM's split products: every element
    within one bf16 step of the fp32 kernel's output (floor 2^-14 of the
    largest), most equal to its rounding, within 2^-8 of the oracle; amp 4
    spreads the scores so that rows rescale mid-walk, and there the bar is
    the oracle's alone at 2^-6."""
    q = normal(770 + rows, (slices, rows, hd)) * np.float32(amp)
    k, v = normal(771 + keys, (slices, keys, hd)), normal(772, (slices, keys, hd))
    mask = _test_mask(kind, rows, keys)
    scale = float(np.float32(1 / np.sqrt(hd)))
    qd, kd, vd, md = dev_f32(q), dev_f32(k), dev_f32(v), dev_f32(mask)
    out = torch.empty(slices, rows, hd, device="cuda")
    backend.attention(qd, kd, vd, out, slices, rows, keys, hd, scale, md)
    want = torch.empty(slices, rows, hd, dtype=torch.bfloat16, device="cuda")
    backend.round_bf16(out, want)
    ws = torch.empty(backend.attention_masked_workspace_floats(slices, rows, keys, hd), device="cuda")
    got = torch.full((slices, rows, hd), float("nan"), dtype=torch.bfloat16, device="cuda")
    backend.attention_masked(qd, kd, vd, got, slices, rows, keys, hd, scale, md, ws)
    torch.cuda.synchronize()
    got_f = oracle.bf16_to_f32(got.view(torch.int16).cpu().numpy().view(np.uint16)).reshape(slices, rows, hd)
    out_f = host_f32(out)
    dead = ~np.isfinite(mask).any(axis=1)
    assert np.array_equal(got_f[:, dead], np.zeros_like(got_f[:, dead]))
    if amp == 1.0:
        tol = 2.0**-8 * np.abs(out_f) + 2.0**-14 * np.abs(out_f).max()
        assert np.all(np.abs(got_f - out_f) <= tol), float(np.max(np.abs(got_f - out_f) - tol))
        assert np.mean(got.view(torch.int16).cpu().numpy() == want.view(torch.int16).cpu().numpy()) > 0.9
    bar = 2.0**-8 if amp == 1.0 else 2.0**-6
    for s in sorted({0, slices - 1}):
        want_o = oracle.attention_head(q[s], k[s], v[s], mask, scale)
        assert_f32_close(got_f[s], want_o, bar, f"masked split-bf16 attention, {kind} mask, slice {s}")


def test_attention_masked_refuses_what_it_cannot_take(backend):
    q = torch.zeros(1, 64, 128, device="cuda")
    out = torch.empty(1, 64, 128, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(backend.attention_masked_workspace_floats(1, 64, 64, 128), device="cuda")
    mask = torch.zeros(64, 64, device="cuda")
    with pytest.raises(ValueError):  # a workspace one float short
        backend.attention_masked(q, q, q, out, 1, 64, 64, 128, 0.1, mask, ws[:-1])
    with pytest.raises(ValueError):  # mask rows shorter than the keys
        m2 = torch.zeros(64, 60, device="cuda")
        backend.attention_masked(q, q, q, out, 1, 64, 64, 128, 0.1, m2, ws)
    with pytest.raises(ValueError):  # an fp32 out
        backend.attention_masked(q, q, q, q, 1, 64, 64, 128, 0.1, mask, ws)
