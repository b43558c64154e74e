"""GPU parity over seeded random shapes: each case draws its shape, dtype and
layout from its own seed, so the kernels' launch-shape choices (one or
several waves per row, the wide-row path, vector or scalar chunks, one or
two tokens per wave, the workgroup size of elementwise grids) are crossed
with row widths and counts the fixed-shape tests do not name. Every case
runs through the C ABI and is checked against the CPU oracle at the
tolerances of tests/parity.py; the shape is in the test id and in every
assertion message."""

import numpy as np
import pytest

import oracle
from parity import assert_bf16_close, assert_f32_close, dev_bf16, dev_f32, dev_i64, host_bits, host_f32, normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

CASES = 16


@pytest.fixture(scope="module", autouse=True)
def device(backend):
    if not torch.cuda.is_available() or backend.device_count() == 0:
        pytest.skip("no HIP device")
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


def draw_shape(g, max_elems=1 << 22):
    """rows and cols log-uniform over [1, 4096] and [1, 40000], cols a multiple
    of 8 two times in three, with rows * cols capped."""
    rows = int(np.exp(g.uniform(0, np.log(4096))))
    cols = int(np.exp(g.uniform(0, np.log(40000))))
    if g.uniform() < 2 / 3:
        cols = max(8, cols // 8 * 8)
    rows = max(1, min(rows, max_elems // cols))
    return rows, cols


def misaligned(t, g):
    """The same values in a view starting one element past a 16-byte
    boundary, one time in four (the scalar paths)."""
    if g.uniform() >= 0.25:
        return t
    base = torch.empty(t.numel() + 8, dtype=t.dtype, device="cuda")
    v = base[1:1 + t.numel()].view(t.shape)
    v.copy_(t)
    return v


def weights(g, cols):
    return (1 + 0.02 * g.standard_normal(cols)).astype(np.float32)


@pytest.mark.parametrize("case", range(CASES))
@pytest.mark.parametrize("op", ["rms", "add_rms", "layer"])
def test_norms_random_shapes(backend, op, case):
    g = np.random.default_rng(1000 * case + {"rms": 1, "add_rms": 2, "layer": 3}[op])
    rows, cols = draw_shape(g)
    bf = g.uniform() < 0.5
    x = normal(int(g.integers(1 << 30)), (rows, cols), 2.0, float(g.uniform(-1, 1)))
    d = normal(int(g.integers(1 << 30)), (rows, cols))
    w, b = weights(g, cols), (0.02 * g.standard_normal(cols)).astype(np.float32)
    what = f"{op} {'bf16' if bf else 'fp32'} {rows}x{cols}"
    if bf:
        x, d = oracle.f32_to_bf16(x), oracle.f32_to_bf16(d)
        xd, dd = misaligned(dev_bf16(x), g), dev_bf16(d)
        xf, df = oracle.bf16_to_f32(x), oracle.bf16_to_f32(d)
    else:
        xd, dd = misaligned(dev_f32(x), g), dev_f32(d)
        xf, df = x, d
    if op == "rms":
        backend.rms_norm(xd, dev_f32(w), 1e-6)
        want = oracle.rms_norm(xf, w, 1e-6)
        got = xd
    elif op == "layer":
        backend.layer_norm(xd, dev_f32(w), dev_f32(b), 1e-6)
        want = oracle.layer_norm(xf, w, b, 1e-6)
        got = xd
    else:
        h = torch.empty_like(xd)
        backend.add_rms_norm(xd, dd, dev_f32(w), h, 1e-6)
        wx, want = oracle.add_rms_norm(xf, df, w, 1e-6)
        if bf:
            assert np.array_equal(host_bits(xd), oracle.f32_to_bf16(wx)), what + " x'"
        else:
            assert np.array_equal(host_f32(xd), wx), what + " x'"
        got = h
    if bf:
        assert_bf16_close(host_bits(got), want, what)
    else:
        assert_f32_close(host_f32(got), want, 1e-5, what)


@pytest.mark.parametrize("case", range(CASES))
def test_rope_random_shapes(backend, case):
    g = np.random.default_rng(7000 + case)
    # half the cases on head widths whose halves fill 16-byte chunks
    dim = int(g.choice([64, 80, 96, 128, 192, 256])) if g.uniform() < 0.5 else 2 * int(g.integers(1, 257))
    half = dim // 2
    qh, kh = int(g.integers(1, 33)), int(g.integers(0, 9))
    rows = max(1, min(int(np.exp(g.uniform(np.log(16), np.log(12000)))), (1 << 23) // ((qh + kh) * dim)))
    n_page = int(g.integers(0, half + 1)) if g.uniform() < 0.3 else 0
    page_mod = int(g.integers(0, 5))
    bf = g.uniform() < 0.6
    tok = g.integers(-40000, 40000, rows)
    page = g.integers(-50, 50, rows)
    inv_tok = oracle.rope_inv(half - n_page, 1e4) if half > n_page else None
    inv_page = oracle.rope_inv(n_page, 256.0) if n_page else None
    q = normal(int(g.integers(1 << 30)), (rows, qh * dim))
    k = normal(int(g.integers(1 << 30)), (rows, max(kh, 1) * dim))
    what = f"rope {'bf16' if bf else 'fp32'} rows {rows} heads {qh}+{kh} dim {dim} n_page {n_page} mod {page_mod}"
    if bf:
        q, k = oracle.f32_to_bf16(q), oracle.f32_to_bf16(k)
        dq, dk = misaligned(dev_bf16(q), g), dev_bf16(k)
        qf, kf = oracle.bf16_to_f32(q), oracle.bf16_to_f32(k)
    else:
        dq, dk = misaligned(dev_f32(q), g), dev_f32(k)
        qf, kf = q, k
    backend.rope_qk(dq, qh, dk if kh else None, kh, dim, dev_i64(tok), dev_i64(page),
                    dev_f32(inv_tok) if inv_tok is not None else None,
                    dev_f32(inv_page) if inv_page is not None else None, page_mod)
    kw = dict(tok=tok, page=page, inv_tok=inv_tok, inv_page=inv_page, page_mod=page_mod)
    wq = oracle.rope(qf, qh, dim, **kw)
    if bf:
        assert_bf16_close(host_bits(dq), wq, what + " q")
    else:
        assert_f32_close(host_f32(dq), wq, 1e-5, what + " q")
    if kh:
        wk = oracle.rope(kf, kh, dim, **kw)
        if bf:
            assert_bf16_close(host_bits(dk), wk, what + " k")
        else:
            assert_f32_close(host_f32(dk), wk, 1e-5, what + " k")


@pytest.mark.parametrize("case", range(CASES))
def test_activations_random_shapes(backend, case):
    g = np.random.default_rng(9000 + case)
    rows, ffn = draw_shape(g, 1 << 21)
    inp = oracle.f32_to_bf16(normal(int(g.integers(1 << 30)), (rows, 2 * ffn), 3.0))
    out = torch.empty(rows, ffn, dtype=torch.bfloat16, device="cuda")
    backend.swiglu(misaligned(dev_bf16(inp), g), out)
    assert_bf16_close(host_bits(out), oracle.swiglu(oracle.bf16_to_f32(inp)), f"swiglu {rows}x{ffn}")
    n = rows * ffn + int(g.integers(0, 8))
    x = normal(int(g.integers(1 << 30)), n, 3.0)
    xb = oracle.f32_to_bf16(x)
    d = misaligned(dev_bf16(xb), g)
    backend.gelu_erf(d)
    assert_bf16_close(host_bits(d), oracle.gelu_erf(oracle.bf16_to_f32(xb)), f"gelu_erf bf16 n={n}")
    d = misaligned(dev_f32(x), g)
    backend.quick_gelu(d)
    assert_f32_close(host_f32(d), oracle.quick_gelu(x), 1e-6, f"quick_gelu n={n}")


@pytest.mark.parametrize("case", range(CASES))
def test_softmax_random_shapes(backend, case):
    g = np.random.default_rng(11000 + case)
    rows, cols = draw_shape(g)
    batch = int(g.integers(1, 5))
    mrows = max(1, rows // batch)
    x = normal(int(g.integers(1 << 30)), (batch * mrows, cols), 4.0)
    mask = np.where(g.uniform(size=(mrows, cols)) < 0.3, -np.inf, 0.0).astype(np.float32)
    mask[g.uniform(size=mrows) < 0.1] = -np.inf  # some rows fully masked
    scale = float(g.uniform(0.05, 1.0))
    what = f"scale_mask_softmax batch {batch} rows {mrows} cols {cols}"
    # the mask applies to slice-major rows: row (s, r) of x uses mask row r
    d = dev_f32(x)
    backend.scale_mask_softmax_rows(d, scale, dev_f32(mask), batch, mrows, cols)
    want = oracle.softmax_rows(oracle.scale_add_mask(x, scale, mask, batch, mrows, cols))
    assert_f32_close(host_f32(d), want, 1e-5, what)
    d = misaligned(dev_f32(x), g)
    backend.softmax_rows(d)
    assert_f32_close(host_f32(d), oracle.softmax_rows(x), 1e-5, f"softmax_rows {batch * mrows}x{cols}")


@pytest.mark.parametrize("case", range(CASES))
def test_gather_random_shapes(backend, case):
    g = np.random.default_rng(13000 + case)
    vocab = int(g.integers(1, 5000))
    cols = int(np.exp(g.uniform(0, np.log(9000))))
    rows = int(g.integers(0, 300))
    table = oracle.f32_to_bf16(0.02 * g.standard_normal((vocab, cols), dtype=np.float32))
    ids = g.integers(-3, vocab + 3, rows)
    out = torch.empty(rows, cols, device="cuda")
    backend.gather_rows_bf16(dev_bf16(table), dev_i64(ids), out, table_rows=vocab)
    want = oracle.embed(table, np.clip(ids, 0, vocab - 1))
    want[(ids < 0) | (ids >= vocab)] = 0.0  # an id outside the table gives a zero row
    assert np.array_equal(host_f32(out).view(np.uint32), want.view(np.uint32)), f"gather {rows} of {vocab}x{cols}"
