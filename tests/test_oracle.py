"""Pins the CPU oracle (oracle/uocr_oracle.c) before any GPU result is judged
against it:

* the reference's own known answers (tests/ops_test.cpp:26-50,
  tests/dtype_test.cpp:20-28);
* the committed golden vectors in tests/golden/, which the reference's own
  code produced (tests/golden/make_golden.py over oracle/_ref);
* closed forms evaluated in float64 and invariants of each op, chosen so
  that a plausible slip (a dropped eps, a flipped sign, interleaved instead
  of half-split pairs, an fp64 instead of fp32 rope angle, a mean instead of
  a root mean square) fails at least one of them; the last tests plant such
  slips in numpy copies of the oracle and check that the checks reject them;
* bit equality with the reference's ops.cpp / page_rope.cpp compiled into
  oracle/_ref where that library was built (this container).
"""

import math
import os

import numpy as np
import pytest
from scipy.special import erf

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")


def near(a, b, tol=1e-5):
    """ops_test.cpp:16: |a - b| <= tol * max(1, |b|)."""
    return abs(float(a) - float(b)) <= tol * max(1.0, abs(float(b)))


def rng(seed=0):
    return np.random.default_rng(seed)


# ---- bf16 ---------------------------------------------------------------------------


def test_bf16_known_answers(orc):
    # dtype_test.cpp:20-28
    for v in [0.0, -0.0, 1.0, -2.5, 1024.0, 3.0517578e-05]:
        got = orc.bf16_to_f32(orc.f32_to_bf16(np.array([v], np.float32)))[0]
        assert got == np.float32(v) and math.copysign(1, got) == math.copysign(1, v)
    assert orc.bf16_round(np.array([1.0 + 2.0**-8], np.float32))[0] == 1.0  # tie down to even
    assert orc.bf16_round(np.array([1.0 + 3 * 2.0**-8], np.float32))[0] == np.float32(1.0 + 2.0**-6)  # tie up
    assert np.isinf(orc.bf16_round(np.array([np.finfo(np.float32).max], np.float32))[0])
    assert np.isnan(orc.bf16_round(np.array([np.nan], np.float32))[0])


def _bf16_patterns():
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x4000, 0xC000], dtype=np.uint32)
    return (hi[:, None] | lows[None, :]).ravel()


def test_bf16_matches_independent_rounding(orc):
    """Every bf16 upper half with eight lower halves (ties, near-ties, zero,
    all ones) against a rule written independently: the nearer of the two
    bf16 neighbours by float64 distance, the even one on a tie, 2^128 standing
    in for infinity; NaN stays NaN, keeps its sign and gets the quiet bit."""
    bits = _bf16_patterns()
    x = bits.view(np.float32)
    got = orc.f32_to_bf16(x).astype(np.uint32)
    nan = np.isnan(x)
    assert np.all(np.isnan(orc.bf16_to_f32(got[nan].astype(np.uint16))))
    assert np.all((got[nan] & 0x40) != 0)
    assert np.all((got[nan] >> 15) == (bits[nan] >> 31))
    fin = ~nan & np.isfinite(x)
    b, xf = bits[fin], x[fin].astype(np.float64)
    lo = b & 0xFFFF0000
    hi = lo + 0x10000
    lo_v = lo.view(np.float32).astype(np.float64)
    hi_bits_abs = hi & 0x7FFFFFFF
    hi_v = np.where(hi_bits_abs == 0x7F800000, np.copysign(2.0**128, xf), 0.0)
    ok = hi_bits_abs != 0x7F800000
    hi_v[ok] = hi[ok].view(np.float32).astype(np.float64)
    d_lo, d_hi = np.abs(xf - lo_v), np.abs(xf - hi_v)
    even_lo = ((lo >> 16) & 1) == 0
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ~even_lo)
    want = np.where(pick_hi, hi >> 16, lo >> 16)
    assert np.array_equal(got[fin], want)
    inf = np.isinf(x)
    assert np.array_equal(got[inf], bits[inf] >> 16)


def test_bf16_widen_is_shift(orc):
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    w = orc.bf16_to_f32(b)
    assert np.array_equal(w.view(np.uint32), b.astype(np.uint32) << 16)


# ---- norms ----------------------------------------------------------------------------


def test_rms_norm_known_answer(orc):
    # ops_test.cpp:31-34
    y = orc.rms_norm(np.array([[3, 4]], np.float32), np.array([2, 1], np.float32), 0.0)
    r = math.sqrt(12.5)
    assert near(y[0, 0], 6 / r) and near(y[0, 1], 4 / r)


def test_layer_norm_known_answer(orc):
    # ops_test.cpp:26-29
    y = orc.layer_norm(np.array([[1, 2, 3, 4]], np.float32), np.ones(4, np.float32), np.zeros(4, np.float32), 0.0)
    s = math.sqrt(1.25)
    assert near(y[0, 0], -1.5 / s) and near(y[0, 3], 1.5 / s)


def rms_closed_form(x, w, eps):
    x64 = x.astype(np.float64)
    return w.astype(np.float64) * x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)


def ln_closed_form(x, w, b, eps):
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=-1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x64 - mu) / np.sqrt(var + eps) * w.astype(np.float64) + b.astype(np.float64)


def rel(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


@pytest.mark.parametrize("rows,cols,eps", [(9, 300, 1e-6), (64, 2048, 1e-6), (7, 1024, 1e-5), (3, 1, 1e-6)])
def test_rms_norm_closed_form(orc, rows, cols, eps):
    g = rng(rows)
    x = g.standard_normal((rows, cols), dtype=np.float32)
    w = (1 + 0.02 * g.standard_normal(cols)).astype(np.float32)
    y = orc.rms_norm(x, w, eps)
    assert rel(y, rms_closed_form(x, w, eps)) < 1e-6
    ones = orc.rms_norm(x, np.ones(cols, np.float32), eps)
    rms = np.sqrt(np.mean(ones.astype(np.float64) ** 2, axis=-1))
    assert np.allclose(rms, 1.0 / np.sqrt(1.0 + eps / np.mean(x.astype(np.float64) ** 2, axis=-1)), rtol=1e-5)


@pytest.mark.parametrize("rows,cols,eps", [(9, 300, 1e-6), (64, 1024, 1e-6), (5, 768, 1e-5)])
def test_layer_norm_closed_form(orc, rows, cols, eps):
    g = rng(cols)
    x = (3 + 2 * g.standard_normal((rows, cols))).astype(np.float32)
    w = (1 + 0.02 * g.standard_normal(cols)).astype(np.float32)
    b = (0.02 * g.standard_normal(cols)).astype(np.float32)
    y = orc.layer_norm(x, w, b, eps)
    assert rel(y, ln_closed_form(x, w, b, eps)) < 1e-6
    z = orc.layer_norm(x, np.ones(cols, np.float32), np.zeros(cols, np.float32), eps).astype(np.float64)
    assert np.all(np.abs(z.mean(axis=-1)) < 1e-5)
    assert np.allclose(z.var(axis=-1), 1.0, rtol=1e-4)


def test_norms_independent_of_thread_count(orc):
    # ops_test.cpp:108-120: one row, one thread, the same arithmetic.
    g = rng(3)
    x = g.standard_normal((33, 700), dtype=np.float32)
    w = g.standard_normal(700, dtype=np.float32)
    b = g.standard_normal(700, dtype=np.float32)
    orc.set_threads(1)
    r1, l1 = orc.rms_norm(x, w, 1e-6), orc.layer_norm(x, w, b, 1e-6)
    orc.set_threads(7)
    r7, l7 = orc.rms_norm(x, w, 1e-6), orc.layer_norm(x, w, b, 1e-6)
    orc.set_threads(1)
    assert np.array_equal(r1.view(np.uint32), r7.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l7.view(np.uint32))


def test_linear_and_attention_independent_of_thread_count(orc):
    # the reference runs linear and attention_head over rows with
    # parallel_for too (ops.cpp:100,225): a row's values never depend on T
    g = rng(4)
    x = g.standard_normal((37, 96), dtype=np.float32)
    w = g.standard_normal((45, 96), dtype=np.float32)
    b = g.standard_normal(45, dtype=np.float32)
    q = g.standard_normal((29, 16), dtype=np.float32)
    k = g.standard_normal((41, 16), dtype=np.float32)
    v = g.standard_normal((41, 24), dtype=np.float32)
    bias = g.standard_normal((29, 41), dtype=np.float32)
    orc.set_threads(1)
    y1, a1 = orc.linear(x, w, b), orc.attention_head(q, k, v, bias, 0.25)
    orc.set_threads(6)
    y6, a6 = orc.linear(x, w, b), orc.attention_head(q, k, v, bias, 0.25)
    orc.set_threads(1)
    assert np.array_equal(y1.view(np.uint32), y6.view(np.uint32))
    assert np.array_equal(a1.view(np.uint32), a6.view(np.uint32))


# ---- activations -------------------------------------------------------------------------


def test_activation_known_answers(orc):
    # ops_test.cpp:42-50
    g = orc.gelu_erf(np.array([-1, 0, 1], np.float32))
    assert near(g[2], 0.8413447) and near(g[0], -0.1586553) and g[1] == 0
    s = orc.silu(np.array([2], np.float32))
    assert near(s[0], 2 / (1 + math.exp(-2.0)))


def test_gelu_closed_form_and_symmetry(orc):
    x = rng(1).standard_normal(100000, dtype=np.float32) * 3
    y = orc.gelu_erf(x).astype(np.float64)
    x64 = x.astype(np.float64)
    want = 0.5 * x64 * (1 + erf(x64 / math.sqrt(2)))
    assert np.all(np.abs(y - want) <= 1e-6 * np.maximum(1, np.abs(want)))
    # g(x) - g(-x) = x
    yn = orc.gelu_erf(-x).astype(np.float64)
    assert np.all(np.abs((y - yn) - x64) <= 2e-6 * np.maximum(1, np.abs(x64)))


def test_silu_mul_closed_form(orc):
    g = rng(2)
    a = g.standard_normal(100000, dtype=np.float32) * 4
    u = g.standard_normal(100000, dtype=np.float32)
    y = orc.silu_mul(a, u).astype(np.float64)
    a64 = a.astype(np.float64)
    want = a64 / (1 + np.exp(-a64)) * u.astype(np.float64)
    assert np.all(np.abs(y - want) <= 1e-6 * np.maximum(1, np.abs(want)))
    assert np.all(orc.silu_mul(a, np.zeros_like(u)) == 0)


def test_swiglu_is_silu_then_multiply(orc):
    g = rng(4)
    inp = g.standard_normal((17, 2 * 96), dtype=np.float32)
    out = orc.swiglu(inp)
    want = orc.silu_mul(inp[:, :96], inp[:, 96:])
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


def test_add_rms_norm_is_the_reference_chain(orc):
    g = rng(5)
    x = g.standard_normal((12, 2048), dtype=np.float32)
    d = g.standard_normal((12, 2048), dtype=np.float32)
    w = (1 + 0.02 * g.standard_normal(2048)).astype(np.float32)
    xs, h = orc.add_rms_norm(x, d, w, 1e-6)
    assert np.array_equal(xs, x + d)  # one fp32 add per element
    assert np.array_equal(h.view(np.uint32), orc.rms_norm(x + d, w, 1e-6).view(np.uint32))
    assert rel(h, rms_closed_form(x + d, w, 1e-6)) < 1e-6


# ---- rope ------------------------------------------------------------------------------------


def rope_closed_form(x, heads, dim, pos, inv):
    """Half-split rotation of each (i, i + half) pair as a complex number by
    the fp32 angle float32(pos) * inv[i], in float64."""
    half = dim // 2
    v = x.astype(np.float64).reshape(x.shape[0], heads, dim)
    ang = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = v[..., :half], v[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1).reshape(x.shape)


def test_rope_table(orc):
    inv = orc.rope_inv(64, 1e4)
    i = np.arange(64, dtype=np.float64)
    assert np.array_equal(inv, (1.0 / np.power(1e4, i / 64)).astype(np.float32))
    assert inv[0] == 1.0 and abs(inv[63] - 1e4 ** (-63 / 64)) < 1e-9


def test_rope_identity_at_zero(orc):
    x = rng(6).standard_normal((3, 4 * 128), dtype=np.float32)
    inv = orc.rope_inv(64, 1e4)
    y = orc.rope(x, 4, 128, tok=np.zeros(3, np.int64), inv_tok=inv)
    assert np.array_equal(y, x)


def test_rope_closed_form_and_invariants(orc):
    g = rng(7)
    rows, heads, dim = 40, 20, 128
    x = g.standard_normal((rows, heads * dim), dtype=np.float32)
    pos = g.integers(0, 20001, rows).astype(np.int64)
    inv = orc.rope_inv(64, 1e4)
    y = orc.rope(x, heads, dim, tok=pos, inv_tok=inv)
    assert rel(y, rope_closed_form(x, heads, dim, pos, inv)) < 2e-6
    # each (i, i + 64) pair keeps its length
    v, w = x.astype(np.float64).reshape(rows, heads, 2, 64), y.astype(np.float64).reshape(rows, heads, 2, 64)
    assert np.allclose((v**2).sum(axis=2), (w**2).sum(axis=2), rtol=1e-5, atol=1e-6)
    # rope(p) then rope(-p) returns the input
    back = orc.rope(y, heads, dim, tok=-pos, inv_tok=inv)
    assert rel(back, x.astype(np.float64)) < 1e-5


def test_rope_one_coordinate_and_page_axis(orc):
    g = rng(8)
    x = g.standard_normal((1, 2 * 16), dtype=np.float32)
    inv_tok = orc.rope_inv(7, 1e4)
    inv_page = np.array([1.0], np.float32)
    a = orc.rope(x, 2, 16, inv_tok=inv_tok, inv_page=inv_page, page_mod=2, one_tok=300, one_page=3)
    b = orc.rope(x, 2, 16, tok=np.array([300]), page=np.array([3]), inv_tok=inv_tok, inv_page=inv_page, page_mod=2)
    assert np.array_equal(a, b)
    # page 3 folds to 1 and page -1 folds to 1 too
    c = orc.rope(x, 2, 16, tok=np.array([300]), page=np.array([-1]), inv_tok=inv_tok, inv_page=inv_page, page_mod=2)
    assert np.array_equal(a, c)


# ---- gather ------------------------------------------------------------------------------------


def test_embed_is_exact_row_take(orc):
    g = rng(9)
    table = orc.f32_to_bf16(g.standard_normal((50, 64), dtype=np.float32) * 0.02)
    ids = np.array([3, 0, 49, 3], np.int64)
    got = orc.embed(table, ids)
    want = (table.astype(np.uint32) << 16).view(np.float32)[ids]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- golden vectors written by the reference's own code -----------------------------------------


@pytest.fixture(scope="module")
def golden():
    if not os.path.exists(GOLDEN):
        pytest.skip("tests/golden/ref_vectors.npz absent")
    return dict(np.load(GOLDEN, allow_pickle=False))


def test_golden_norms(orc, golden):
    x, w, b = golden["norm_x"], golden["norm_w"], golden["norm_b"]
    eps = float(golden["norm_eps"])
    assert np.array_equal(orc.rms_norm(x, w, eps).view(np.uint32), golden["rms_out"].view(np.uint32))
    assert np.array_equal(orc.layer_norm(x, w, b, eps).view(np.uint32), golden["ln_out"].view(np.uint32))


def test_golden_activations(orc, golden):
    assert np.array_equal(orc.gelu_erf(golden["act_x"]).view(np.uint32), golden["gelu_out"].view(np.uint32))
    assert np.array_equal(orc.silu(golden["act_x"]).view(np.uint32), golden["silu_out"].view(np.uint32))


def test_golden_rope(orc, golden):
    dim, heads = int(golden["rope_dim"]), int(golden["rope_heads"])
    inv_tok, inv_page = golden["rope_inv_tok"], golden["rope_inv_page"]
    assert np.array_equal(orc.rope_inv(inv_tok.size, float(golden["rope_tok_theta"])), inv_tok)
    assert np.array_equal(orc.rope_inv(inv_page.size, float(golden["rope_page_theta"])), inv_page)
    y = orc.rope(golden["rope_x"], heads, dim, tok=golden["rope_tok"], page=golden["rope_page"], inv_tok=inv_tok,
                 inv_page=inv_page, page_mod=int(golden["rope_page_mod"]))
    assert np.array_equal(y.view(np.uint32), golden["rope_out"].view(np.uint32))


def test_golden_bf16(orc, golden):
    assert np.array_equal(orc.f32_to_bf16(golden["bf16_in"].view(np.float32)), golden["bf16_out"])


# ---- the live reference (this container only) ----------------------------------------------------


@pytest.fixture(scope="module")
def ref(orc):
    r = orc.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return r


def _p(a):
    return None if a is None else a.ctypes.data


def test_oracle_bit_equals_reference_norms_and_activations(orc, ref):
    g = rng(10)
    for rows, cols in [(9, 300), (33, 2048), (4, 1024), (2, 7)]:
        x = g.standard_normal((rows, cols), dtype=np.float32)
        w = g.standard_normal(cols, dtype=np.float32)
        b = g.standard_normal(cols, dtype=np.float32)
        r1 = x.copy()
        ref.ref_rms_norm(_p(r1), _p(w), rows, cols, np.float32(1e-6))
        assert np.array_equal(r1.view(np.uint32), orc.rms_norm(x, w, 1e-6).view(np.uint32))
        r2 = x.copy()
        ref.ref_layer_norm(_p(r2), _p(w), _p(b), rows, cols, np.float32(1e-6))
        assert np.array_equal(r2.view(np.uint32), orc.layer_norm(x, w, b, 1e-6).view(np.uint32))
        r3 = x.copy() * 3
        ref.ref_gelu_erf(_p(r3), r3.size)
        assert np.array_equal(r3.view(np.uint32), orc.gelu_erf(x * 3).view(np.uint32))
        r4 = x.copy() * 3
        ref.ref_silu(_p(r4), r4.size)
        assert np.array_equal(r4.view(np.uint32), orc.silu(x * 3).view(np.uint32))


def test_oracle_bit_equals_reference_rope(orc, ref):
    g = rng(11)
    for dim, pairs, heads in [(128, 1, 10), (16, 1, 2), (64, 3, 1)]:
        half = dim // 2
        inv_tok = np.empty(half - pairs, np.float32)
        inv_page = np.empty(pairs, np.float32)
        ref.ref_rope_tables(dim, 1e4, 256.0, pairs, _p(inv_tok), _p(inv_page))
        assert np.array_equal(inv_tok, orc.rope_inv(half - pairs, 1e4))
        assert np.array_equal(inv_page, orc.rope_inv(pairs, 256.0))
        rows = 37
        x = g.standard_normal((rows, heads * dim), dtype=np.float32)
        tok = g.integers(0, 30000, rows).astype(np.int64)
        page = g.integers(-5, 9, rows).astype(np.int64)
        want = x.copy()
        ref.ref_rope_apply(_p(want), rows, heads * dim, dim, 1e4, 256.0, pairs, 2, _p(tok), _p(page))
        got = orc.rope(x, heads, dim, tok=tok, page=page, inv_tok=inv_tok, inv_page=inv_page, page_mod=2)
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32))


def test_oracle_bit_equals_reference_bf16(orc, ref):
    bits = _bf16_patterns()
    x = bits.view(np.float32)
    want = np.array([ref.ref_f32_to_bf16(np.float32(v)) for v in x[::97]], np.uint16)
    assert np.array_equal(orc.f32_to_bf16(x[::97]), want)


# ---- the checks reject planted slips ----------------------------------------------------------------


def test_checks_reject_planted_slips(orc):
    """Slips planted in numpy copies of the oracle's formulas fail the checks
    above, so those checks pin more than a retyped formula would."""
    g = rng(12)
    x = g.standard_normal((8, 256), dtype=np.float32)
    w = (1 + 0.02 * g.standard_normal(256)).astype(np.float32)
    # rms over the mean instead of the mean square
    slip = w * x / np.sqrt(np.abs(x.mean(axis=-1, keepdims=True)) + 1e-6)
    assert rel(slip, rms_closed_form(x, w, 1e-6)) > 1e-3
    # eps dropped: visible on a row of tiny values
    tiny = np.full((1, 256), 1e-4, np.float32)
    no_eps = w * tiny / np.sqrt(np.mean(tiny.astype(np.float64) ** 2))
    assert rel(no_eps, rms_closed_form(tiny, w, 1e-6)) > 1e-3
    # rope: flipped sin sign, interleaved pairs, fp64 angle
    rows, heads, dim = 8, 2, 128
    xr = g.standard_normal((rows, heads * dim), dtype=np.float32)
    pos = g.integers(10000, 20001, rows).astype(np.int64)
    inv = orc.rope_inv(64, 1e4)
    truth = rope_closed_form(xr, heads, dim, pos, inv)
    v = xr.astype(np.float64).reshape(rows, heads, dim)
    ang = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = v[..., :64], v[..., 64:]
    flipped = np.concatenate([a * c + b * s, b * c - a * s], axis=-1).reshape(xr.shape)
    assert rel(flipped, truth) > 1e-2
    ai, bi = v[..., 0::2], v[..., 1::2]
    inter = np.stack([ai * c - bi * s, bi * c + ai * s], axis=-1).reshape(xr.shape)
    assert rel(inter, truth) > 1e-2
    ang64 = pos.astype(np.float64)[:, None] * inv.astype(np.float64)[None, :]
    c64, s64 = np.cos(ang64)[:, None, :], np.sin(ang64)[:, None, :]
    wide = np.concatenate([a * c64 - b * s64, b * c64 + a * s64], axis=-1).reshape(xr.shape)
    assert rel(wide, truth) > 2e-6


# ---- the decode-step neighbours and the row ops beside the path -------------------------------------


def test_router_norm_closed_form_and_edges(orc):
    g = rng(20)
    x = g.standard_normal((6, 320), dtype=np.float32) * 3
    w = (0.1 * g.standard_normal(320)).astype(np.float32)
    y = orc.router_norm(x, w, 1e-6).astype(np.float64)
    x64 = x.astype(np.float64)
    n = x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + 1e-6)
    want = np.clip(np.clip(n, -1e4, 1e4) * (1 + w.astype(np.float64)), -1e4, 1e4)
    assert rel(y, want) < 1e-6
    # non-finite inputs count as zero; huge gains clamp at 1e4
    bad = x[:2].copy()
    bad[0, 5], bad[1, 7], bad[1, 8] = np.nan, np.inf, -np.inf
    yb = orc.router_norm(bad, w, 1e-6)
    clean = bad.copy()
    clean[~np.isfinite(clean)] = 0
    assert np.array_equal(yb, orc.router_norm(clean, w, 1e-6))
    assert np.all(np.isfinite(yb))
    big = orc.router_norm(x[:1], np.full(320, 1e6, np.float32), 1e-6)
    assert np.all(np.abs(big) <= 1e4) and np.any(np.abs(big) == 1e4)


def test_softmax_known_answer_and_masking(orc):
    # ops_test.cpp:51-55
    sm = orc.softmax_rows(np.array([[0, 0, math.log(2.0)], [-np.inf] * 3], np.float32))
    assert near(sm[0, 0], 0.25) and near(sm[0, 2], 0.5)
    assert sm[1, 0] == 0 and sm[1, 2] == 0
    x = rng(21).standard_normal((9, 500), dtype=np.float32) * 4
    y = orc.softmax_rows(x).astype(np.float64)
    assert np.allclose(y.sum(axis=1), 1.0, atol=1e-6)
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    assert rel(y, e / e.sum(axis=1, keepdims=True)) < 1e-6


def test_linear_closed_form(orc):
    g = rng(22)
    x = g.standard_normal((4, 1280), dtype=np.float32)
    w = (0.05 * g.standard_normal((96, 1280))).astype(np.float32)
    b = g.standard_normal(96, dtype=np.float32)
    y = orc.linear(x, w, b)
    assert rel(y, x.astype(np.float64) @ w.astype(np.float64).T + b) < 1e-6


def test_attention_known_answers_and_closed_form(orc):
    # ops_test.cpp:68-77: a masked second key leaves the first value; a zero
    # query averages the values.
    k = np.array([[1, 0], [0, 1]], np.float32)
    v = np.array([[5, 6], [7, 8]], np.float32)
    out = orc.attention_one(np.array([1, 0], np.float32), k, v, 1, 2, bias=np.array([0, -np.inf], np.float32))
    assert near(out[0], 5) and near(out[1], 6)
    even = orc.attention_one(np.zeros(2, np.float32), k, v, 1, 2)
    assert near(even[0], 6) and near(even[1], 7)
    # all keys masked: zeros
    assert np.all(orc.attention_one(np.ones(2, np.float32), k, v, 1, 2,
                                    bias=np.full(2, -np.inf, np.float32)) == 0)
    g = rng(23)
    heads, hd, keys = 3, 64, 77
    q = g.standard_normal(heads * hd, dtype=np.float32)
    kk = g.standard_normal((keys, heads * hd), dtype=np.float32)
    vv = g.standard_normal((keys, heads * hd), dtype=np.float32)
    mask = np.where(g.random(keys) < 0.3, -np.inf, 0).astype(np.float32)
    got = orc.attention_one(q, kk, vv, heads, hd, bias=mask, scale=0.125)
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        s = kk[:, sl].astype(np.float64) @ q[sl].astype(np.float64) * 0.125 + mask
        p = np.exp(s - s.max())
        p /= p.sum()
        assert rel(got[sl], p @ vv[:, sl].astype(np.float64)) < 1e-5


def test_scale_add_mask_elementwise(orc):
    g = rng(24)
    x = g.standard_normal((2, 5, 7), dtype=np.float32)
    m = g.standard_normal((5, 7), dtype=np.float32)
    got = orc.scale_add_mask(x, 0.5, m, 2, 5, 7)
    assert np.array_equal(got, (x * np.float32(0.5) + m[None]).astype(np.float32))
    assert np.array_equal(orc.scale_add_mask(x, 2.0, None, 2, 5, 7), x * np.float32(2.0))


def test_quick_gelu_known_answer(orc):
    # ops_test.cpp:44-46
    assert near(orc.quick_gelu(np.array([1.0], np.float32))[0], 1 / (1 + math.exp(-1.702)))


def test_golden_row_ops(orc, golden):
    assert np.array_equal(orc.softmax_rows(golden["softmax_in"]).view(np.uint32), golden["softmax_out"].view(np.uint32))
    assert np.array_equal(orc.linear(golden["linear_x"], golden["linear_w"], golden["linear_b"]).view(np.uint32),
                          golden["linear_y"].view(np.uint32))
    ao = orc.attention_one(golden["attn_q"][0], golden["attn_k"], golden["attn_v"], 1, 64,
                           bias=golden["attn_mask"][0], scale=float(golden["attn_scale"]))
    assert np.array_equal(ao.view(np.uint32), golden["attn_out"][0].view(np.uint32))
    assert np.array_equal(orc.quick_gelu(golden["act_x"]).view(np.uint32), golden["quick_gelu_out"].view(np.uint32))


def test_oracle_bit_equals_reference_row_ops(orc, ref):
    g = rng(25)
    x = (g.standard_normal((7, 1000)) * 5).astype(np.float32)
    x[1, ::7] = -np.inf
    x[4, :] = -np.inf
    r = x.copy()
    ref.ref_softmax_rows(_p(r), 7, 1000)
    assert np.array_equal(r.view(np.uint32), orc.softmax_rows(x).view(np.uint32))
    lx = g.standard_normal((5, 1283), dtype=np.float32)
    lw = g.standard_normal((33, 1283), dtype=np.float32)
    ly = np.empty((5, 33), np.float32)
    ref.ref_linear(_p(lx), 5, 1283, _p(lw), 33, None, _p(ly))
    assert np.array_equal(ly.view(np.uint32), orc.linear(lx, lw).view(np.uint32))
    heads, hd, keys = 2, 128, 300
    q = g.standard_normal(heads * hd, dtype=np.float32)
    kk = g.standard_normal((keys, heads * hd), dtype=np.float32)
    vv = g.standard_normal((keys, heads * hd), dtype=np.float32)
    mask = np.where(g.random(keys) < 0.4, -np.inf, 0).astype(np.float32)
    mine = orc.attention_one(q, kk, vv, heads, hd, bias=mask, scale=0.088)
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        qh, kh, vh = np.ascontiguousarray(q[sl][None]), np.ascontiguousarray(kk[:, sl]), np.ascontiguousarray(vv[:, sl])
        o = np.empty((1, hd), np.float32)
        ref.ref_attention_head(_p(qh), 1, _p(kh), keys, hd, _p(vh), hd, _p(np.ascontiguousarray(mask[None])),
                               np.float32(0.088), _p(o))
        assert np.array_equal(o[0].view(np.uint32), mine[sl].view(np.uint32))
    qx = x[0] * 0.3
    r2 = qx.copy()
    ref.ref_quick_gelu(_p(r2), r2.size)
    assert np.array_equal(r2.view(np.uint32), orc.quick_gelu(qx).view(np.uint32))


def test_expert_topk_known_answer_ties_and_brute_force(orc):
    """The routing rule of src/model/feed_forward.cpp:36-53: softmax, then
    the k top scores with the lower index first on a tie."""
    ids, w = orc.expert_topk(np.array([[1.0, 2.0, 3.0, 2.0]], np.float32), 3)
    assert ids.tolist() == [[2, 1, 3]]  # 1 and 3 tie: the lower index first
    e = np.exp(np.array([1.0, 2.0, 3.0, 2.0]) - 3.0)
    assert np.allclose(w[0], (e / e.sum())[[2, 1, 3]], rtol=1e-6)
    # equal logits: every score ties, so the ids come out in index order
    ids, w = orc.expert_topk(np.zeros((1, 7), np.float32), 7)
    assert ids.tolist() == [list(range(7))] and np.allclose(w, 1 / 7)
    # a row of -inf logits scores every expert 0 (softmax_rows' masked row)
    ids, w = orc.expert_topk(np.full((1, 5), -np.inf, np.float32), 2)
    assert ids.tolist() == [[0, 1]] and not w.any()
    # brute force: a stable sort on (-score, index) over the oracle's own scores
    g = np.random.default_rng(77)
    logits = g.standard_normal((40, 64)).astype(np.float32)
    logits[:, 10] = logits[:, 11] = 5.0  # an exact tie at the top of every row
    ids, w = orc.expert_topk(logits, 6)
    scores = orc.softmax_rows(logits.copy())
    for r in range(40):
        order = sorted(range(64), key=lambda e: (-scores[r, e], e))[:6]
        assert ids[r].tolist() == order and np.array_equal(w[r], scores[r, order])
        assert ids[r, :2].tolist() == [10, 11]
    # a planted slip (ties to the higher index) fails the same check
    slip = sorted(range(64), key=lambda e: (-scores[0, e], -e))[:6]
    assert slip != ids[0].tolist()


# ---- the block router (src/model/block_router.cpp, attention_plan.cpp, decoder.cpp:42-56) -------


def test_entmax15_known_answers_and_invariants(orc):
    # two equal scores split the mass; a far-ahead score takes all of it
    assert np.allclose(orc.entmax15(np.array([0.0, 0.0], np.float32)), [0.5, 0.5], rtol=0, atol=1e-7)
    assert orc.entmax15(np.array([10.0, 0.0], np.float32)).tolist() == [1.0, 0.0]
    assert orc.entmax15(np.array([3.0], np.float32)).tolist() == [1.0]
    g = rng(60)
    for n in (2, 5, 16, 32):
        for _ in range(20):
            x = (g.standard_normal(n) * 3).astype(np.float32)
            p = orc.entmax15(x)
            assert np.all(p >= 0) and abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5
            # order-preserving and shift-invariant, and p = max((x - max)/2 - tau, 0)^2 for one tau
            assert np.all(np.diff(p[np.argsort(-x, kind="stable")]) <= 0)
            assert np.array_equal(orc.entmax15(x + np.float32(4.0)), p) or np.allclose(orc.entmax15(x + 4), p, atol=1e-6)
            h = (x.astype(np.float64) - x.max()) / 2
            on = p > 0
            taus = h[on] - np.sqrt(p[on].astype(np.float64))
            assert np.ptp(taus) < 1e-5 and np.all(h[~on] <= taus.mean() + 1e-6)


def test_block_summaries_known_answers_and_closed_form(orc):
    g = rng(61)
    d, bs = 16, 4
    rk = g.standard_normal((10, d), dtype=np.float32)
    cls = g.standard_normal(d, dtype=np.float32)
    s = orc.block_summaries(rk, cls, bs)
    assert s.shape == (3, d)
    one = orc.block_summaries(rk[:9], cls, bs)  # a one-key last block summarises to that key
    assert np.array_equal(one[2], rk[8])
    for b in range(3):  # fp64 closed form: the softmax(clamp(rk . cls / sqrt d))-weighted mean
        rows = rk[b * bs:(b + 1) * bs].astype(np.float64)
        a = np.clip(rows @ cls.astype(np.float64) / np.sqrt(d), -1e4, 1e4)
        w = np.exp(a - a.max())
        want = (w / w.sum()) @ rows
        assert np.max(np.abs(s[b] - want)) < 1e-5


def test_block_scores_mask_the_local_window(orc):
    g = rng(62)
    d = 8
    S = g.standard_normal((20, d), dtype=np.float32)
    rq = g.standard_normal((3, d), dtype=np.float32)
    z = orc.block_scores(rq, S, [0, 160, 639], 32, 4)
    assert np.all(z[0] == -1e9)  # pos 0: no block before the window
    assert np.all(z[1, 2:] == -1e9) and np.all(z[1, :2] != -1e9)  # pos 160: blocks 0 and 1 (160 // 32 - 4 = 1)
    assert np.all(z[2, 16:] == -1e9)  # pos 639: blocks 0..15
    want = np.clip(rq[2].astype(np.float64) @ S[:16].T.astype(np.float64) / np.sqrt(d), -1e4, 1e4)
    assert np.max(np.abs(z[2, :16] - want)) < 1e-5


def test_select_and_mask_known_answer(orc):
    p = orc.RouterParams(top_m=4, top_k=2, idx_scale=1.0)
    # three remote blocks, one clear winner; block 3 masked
    scores = np.array([[0.0, 9.0, 0.0, -1e9]], np.float32)
    block, bias, valid = orc.select_blocks(scores, None, p)
    assert block.tolist() == [[1, 0]] and valid.tolist() == [[1, 1]]
    # entmax over (9, 0, 0, -1e4) puts all mass on block 1: log(1) and log(floor)
    lp = [0.0, float(np.log(np.float32(1e-4)))]
    mu = (lp[0] + lp[1]) / 2
    assert np.allclose(bias[0], [lp[0] - mu, lp[1] - mu], rtol=1e-6)
    # the key mask of that selection for a query at pos 255 over 256 keys
    m = orc.key_mask(block, bias, valid, 255, 256, p)[0]
    assert np.all(m[128:] == 0)  # the local window (4 blocks of 32)
    assert np.all(m[32:64] == bias[0, 0]) and np.all(m[0:32] == bias[0, 1])
    assert np.all(m[64:128] == -np.inf)
    # a candidate list that excludes every remote block falls back to all of them
    b2, _, v2 = orc.select_blocks(scores, np.array([[0, 0, 0, 1]], np.uint8), p)
    assert b2.tolist() == [[1, 0]] and v2.tolist() == [[1, 1]]
    # a candidate list keeps only its blocks valid (ties: the lower index first)
    b3, _, v3 = orc.select_blocks(np.array([[5.0, 5.0, 5.0, -1e9]], np.float32), np.array([[0, 1, 1, 0]], np.uint8), p)
    assert b3.tolist() == [[1, 2]] and v3.tolist() == [[1, 1]]


def test_page_candidates_known_answers(orc):
    lo, hi = [0, 0, 1, -1, 2], [0, 1, 2, -1, 2]
    assert orc.page_candidates(lo, hi, -1, 5) is None  # no page: no restriction
    assert orc.page_candidates(lo, hi, 1, 5).tolist() == [0, 1, 1, 0, 0]
    assert orc.page_candidates(lo, hi, 2, 7).tolist() == [0, 0, 1, 0, 1, 0, 0]
    assert orc.page_candidates(lo, hi, 9, 5) is None  # no block holds the page
    assert orc.page_candidates(lo, hi, 2, 3).tolist() == [0, 0, 1]  # only the first nblk blocks count


def test_oracle_bit_equals_reference_router(orc, ref):
    g = rng(63)
    d = 128
    for keys in (1, 31, 32, 33, 300, 1025):
        rk = (g.standard_normal((keys, d)) * 3).astype(np.float32)
        cls = g.standard_normal(d, dtype=np.float32)
        mine = orc.block_summaries(rk, cls, 32)
        theirs = np.empty_like(mine)
        ref.ref_block_summaries(_p(rk), keys, d, _p(cls), 32, _p(theirs))
        assert np.array_equal(mine.view(np.uint32), theirs.view(np.uint32)), keys
        rq = g.standard_normal((3, d), dtype=np.float32) * 2
        pos = np.array([keys - 1, keys // 2, 0], np.int64)
        z = orc.block_scores(rq, mine, pos, 32, 4)
        zt = np.empty_like(z)
        ref.ref_block_scores(_p(rq), 3, _p(mine), mine.shape[0], d, _p(pos), 32, 4, _p(zt))
        assert np.array_equal(z.view(np.uint32), zt.view(np.uint32))
    for n in (1, 2, 3, 16, 32):
        for _ in range(10):
            x = (g.standard_normal(n) * 4).astype(np.float32)
            x[g.random(n) < 0.2] = -1e4
            t = x.copy()
            ref.ref_entmax15(_p(t), n)
            assert np.array_equal(orc.entmax15(x).view(np.uint32), t.view(np.uint32))
    for nblk, cand_kind in ((1, None), (7, None), (40, None), (40, "some"), (40, "no remote"), (300, "some")):
        p = orc.RouterParams()
        lq = 4
        scores = (g.standard_normal((lq, nblk)) * 3).astype(np.float32)
        scores[:, nblk // 2:] = -1e9  # the window and beyond
        scores[1, :3] = 2.5  # exact ties
        cand = None
        if cand_kind == "some":
            cand = (g.random((lq, nblk)) < 0.3).astype(np.uint8)
        elif cand_kind == "no remote":
            cand = np.zeros((lq, nblk), np.uint8)
            cand[:, nblk // 2:] = 1
        block, bias, valid = orc.select_blocks(scores, cand, p)
        cap = lq * p.top_k
        tb, tbias, tv = np.empty(cap, np.int64), np.empty(cap, np.float32), np.empty(cap, np.uint8)
        w = ref.ref_select_blocks(_p(scores), lq, nblk, _p(cand), p.top_m, p.top_k, p.idx_scale, p.floor, p.sigma,
                                  _p(tb), _p(tbias), _p(tv))
        assert w == block.shape[1]
        assert np.array_equal(block.ravel(), tb[:lq * w]) and np.array_equal(valid.ravel(), tv[:lq * w])
        assert np.array_equal(bias.ravel().view(np.uint32), tbias[:lq * w].view(np.uint32))
        keys = nblk * 32 - 5
        for first in (0, keys - lq):
            m = orc.key_mask(block, bias, valid, first, keys, p)
            tm = np.empty_like(m)
            ref.ref_key_mask(_p(block), _p(bias), _p(valid), w, lq, first, keys, 32, 4, _p(tm))
            assert np.array_equal(m.view(np.uint32), tm.view(np.uint32))


def test_golden_router(orc, golden):
    if "router_rk" not in golden:
        pytest.skip("golden vectors predate the router")
    p = orc.RouterParams()
    s = orc.block_summaries(golden["router_rk"], golden["router_cls"], 32)
    assert np.array_equal(s.view(np.uint32), golden["router_summaries"].view(np.uint32))
    z = orc.block_scores(golden["router_rq"], s, golden["router_pos"], 32, 4)
    assert np.array_equal(z.view(np.uint32), golden["router_scores"].view(np.uint32))
    block, bias, valid = orc.select_blocks(z, golden["router_cand"], p)
    assert np.array_equal(block, golden["router_block"]) and np.array_equal(valid, golden["router_valid"])
    assert np.array_equal(bias.view(np.uint32), golden["router_bias"].view(np.uint32))
    m = orc.key_mask(block, bias, valid, int(golden["router_first"]), int(golden["router_keys"]), p)
    assert np.array_equal(m.view(np.uint32), golden["router_mask"].view(np.uint32))
    assert np.array_equal(orc.entmax15(golden["entmax_in"]).view(np.uint32), golden["entmax_out"].view(np.uint32))


def test_router_checks_reject_planted_slips(orc):
    """Numpy copies of the selection with a planted slip fail the oracle's own
    answers: ties to the higher index, a softmax instead of entmax, the bias
    without the mean subtracted."""
    p = orc.RouterParams(top_m=8, top_k=4, idx_scale=1.0)
    g = rng(64)
    z = (g.standard_normal((1, 20)) * 2).astype(np.float32)
    z[0, 3] = z[0, 7] = np.float32(4.0)
    block, bias, valid = orc.select_blocks(z, None, p)
    assert block[0, :2].tolist() == [3, 7]
    slip_ties = sorted(range(20), key=lambda b: (-z[0, b], -b))[:4]
    assert slip_ties != block[0].tolist()
    top = np.sort(z[0])[::-1][:8].astype(np.float32)
    soft = np.exp(top - top.max()) / np.exp(top - top.max()).sum()
    assert not np.allclose(orc.entmax15(top), soft, atol=1e-3)
    logp = np.log(np.maximum(orc.entmax15(top)[:4], np.float32(1e-4)))
    assert not np.allclose(bias[0], logp, atol=1e-3) and np.allclose(bias[0], logp - logp.mean(), atol=1e-5)
