"""GPU parity on tensors past 2^31 elements (4-17 GB each), the sizes one
MI355X's 288 GB of HBM holds: every element offset above 2^31 (and byte
offset above 2^32) must be formed in 64 bits.

The inputs repeat with a period that does not divide any power of two (7
rows, or 65544 elements for the flat op), so an offset that wrapped or was
truncated would read or write an element of another phase, and an element
left unwritten would still hold its input. Each op first runs on one period,
checked against the oracle at the tolerances of tests/parity.py; every
period of the large run must then equal that result bitwise (the kernels
fix their reduction order by the row width alone, so a row's result does not
depend on the row count). The attention and the gather are checked against
the oracle directly. The comparisons of the large outputs run on the device
(torch, as plumbing)."""

import numpy as np
import pytest

import oracle
from parity import assert_bf16_close, assert_f32_close, dev_bf16, dev_f32, dev_i64, host_bits, host_f32, normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

PERIOD = 7
TWO31 = 1 << 31


@pytest.fixture(scope="module", autouse=True)
def device(backend):
    if not torch.cuda.is_available() or backend.device_count() == 0:
        pytest.skip("no HIP device")
    torch.cuda.set_device(0)
    if torch.cuda.get_device_properties(0).total_memory < 64 << 30:
        pytest.skip("needs 64 GB of device memory")
    yield
    torch.cuda.synchronize()


@pytest.fixture(autouse=True)
def release():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def tiled(base, rows):
    """[rows, cols] with row r = base[r % len(base)], built on the device."""
    p, cols = base.shape
    out = torch.empty(rows, cols, dtype=base.dtype, device="cuda")
    q, t = divmod(rows, p)
    out[:q * p].view(q, p, cols).copy_(base.unsqueeze(0).expand(q, p, cols))
    out[q * p:].copy_(base[:t])
    return out


def bits(t):
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def assert_periodic(out, want, what):
    """Every row r of out [rows, cols] bitwise equal to want[r % len(want)]."""
    p = want.shape[0]
    wb, ob = bits(want), bits(out)
    for i in range(p):
        bad = (ob[i::p] != wb[i]).any(dim=1).nonzero()
        assert bad.numel() == 0, f"{what}: row {i + p * int(bad[0, 0])} of {out.shape[0]} differs from the one-period run"


def test_gelu_bf16_past_2_31_elements(backend):
    period = 65544  # 8-element chunks, not a divisor of 2^31
    n = TWO31 + 40
    base = oracle.f32_to_bf16(normal(900, period, 3.0))
    small = dev_bf16(base)
    backend.gelu_erf(small)
    assert_bf16_close(host_bits(small), oracle.gelu_erf(oracle.bf16_to_f32(base)), "gelu one period")
    x = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    m = n // period
    x[:m * period].view(m, period).copy_(dev_bf16(base).unsqueeze(0).expand(m, period))
    x[m * period:].copy_(dev_bf16(base)[:n - m * period])
    backend.gelu_erf(x)
    assert_periodic(x[:m * period].view(m, period), small.view(1, period), f"gelu_erf bf16 n={n}")
    assert torch.equal(bits(x[m * period:]), bits(small[:n - m * period])), "gelu_erf bf16 tail"


def test_swiglu_bf16_past_2_31_elements(backend):
    ffn = 1408
    rows = TWO31 // (2 * ffn) + 13
    base = oracle.f32_to_bf16(normal(901, (PERIOD, 2 * ffn), 3.0))
    small = torch.empty(PERIOD, ffn, dtype=torch.bfloat16, device="cuda")
    backend.swiglu(dev_bf16(base), small)
    assert_bf16_close(host_bits(small), oracle.swiglu(oracle.bf16_to_f32(base)), "swiglu one period")
    inp = tiled(dev_bf16(base), rows)
    out = torch.empty(rows, ffn, dtype=torch.bfloat16, device="cuda")
    backend.swiglu(inp, out)
    assert_periodic(out, small, f"swiglu bf16 [{rows}, 2 x {ffn}]")


def test_add_rms_norm_bf16_past_2_31_elements(backend):
    cols = 2048
    rows = TWO31 // cols + 3
    x = oracle.f32_to_bf16(normal(902, (PERIOD, cols), 2.0))
    d = oracle.f32_to_bf16(normal(903, (PERIOD, cols)))
    w = dev_f32(1 + 0.02 * normal(904, cols))
    sx, sh = dev_bf16(x), torch.empty(PERIOD, cols, dtype=torch.bfloat16, device="cuda")
    backend.add_rms_norm(sx, dev_bf16(d), w, sh, 1e-6)
    wx, wh = oracle.add_rms_norm(oracle.bf16_to_f32(x), oracle.bf16_to_f32(d), host_f32(w), 1e-6)
    assert np.array_equal(host_bits(sx), oracle.f32_to_bf16(wx)), "add_rms_norm x' one period"
    assert_bf16_close(host_bits(sh), wh, "add_rms_norm h one period")
    lx, ld = tiled(dev_bf16(x), rows), tiled(dev_bf16(d), rows)
    lh = torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda")
    backend.add_rms_norm(lx, ld, w, lh, 1e-6)
    del ld
    assert_periodic(lx, sx, f"add_rms_norm bf16 x' [{rows}, {cols}]")
    assert_periodic(lh, sh, f"add_rms_norm bf16 h [{rows}, {cols}]")


def test_rms_norm_f32_past_2_31_elements(backend):
    cols = 4096
    rows = TWO31 // cols + 5
    x = normal(905, (PERIOD, cols), 2.0)
    w = dev_f32(1 + 0.02 * normal(906, cols))
    small = dev_f32(x)
    backend.rms_norm(small, w, 1e-6)
    assert_f32_close(host_f32(small), oracle.rms_norm(x, host_f32(w), 1e-6), 1e-5, "rms_norm one period")
    big = tiled(dev_f32(x), rows)
    backend.rms_norm(big, w, 1e-6)
    assert_periodic(big, small, f"rms_norm f32 [{rows}, {cols}]")


def test_layer_norm_bf16_past_2_31_elements(backend):
    cols = 1024
    rows = TWO31 // cols + 1
    x = oracle.f32_to_bf16(normal(907, (PERIOD, cols), 2.0, 0.5))
    w, b = dev_f32(1 + 0.02 * normal(908, cols)), dev_f32(0.02 * normal(909, cols))
    small = dev_bf16(x)
    backend.layer_norm(small, w, b, 1e-6)
    assert_bf16_close(host_bits(small), oracle.layer_norm(oracle.bf16_to_f32(x), host_f32(w), host_f32(b), 1e-6),
                      "layer_norm one period")
    big = tiled(dev_bf16(x), rows)
    backend.layer_norm(big, w, b, 1e-6)
    assert_periodic(big, small, f"layer_norm bf16 [{rows}, {cols}]")


def test_rope_qk_bf16_past_2_31_elements(backend):
    qh, kh, dim = 16, 4, 128
    rows = TWO31 // (qh * dim) + 7
    q = oracle.f32_to_bf16(normal(910, (PERIOD, qh * dim)))
    k = oracle.f32_to_bf16(normal(911, (PERIOD, kh * dim)))
    pos = np.arange(PERIOD, dtype=np.int64) * 911
    inv = oracle.rope_inv(dim // 2, 1e4)
    sq, sk = dev_bf16(q), dev_bf16(k)
    backend.rope_qk(sq, qh, sk, kh, dim, dev_i64(pos), None, dev_f32(inv), None, 0)
    assert_bf16_close(host_bits(sq), oracle.rope(oracle.bf16_to_f32(q), qh, dim, tok=pos, inv_tok=inv),
                      "rope q one period")
    assert_bf16_close(host_bits(sk), oracle.rope(oracle.bf16_to_f32(k), kh, dim, tok=pos, inv_tok=inv),
                      "rope k one period")
    lq, lk = tiled(dev_bf16(q), rows), tiled(dev_bf16(k), rows)
    lpos = tiled(dev_i64(pos).view(PERIOD, 1), rows).view(rows)
    backend.rope_qk(lq, qh, lk, kh, dim, lpos, None, dev_f32(inv), None, 0)
    assert_periodic(lq, sq, f"rope q bf16 [{rows}, {qh} x {dim}]")
    assert_periodic(lk, sk, f"rope k bf16 [{rows}, {kh} x {dim}]")


def test_softmax_rows_f32_past_2_31_elements(backend):
    cols = 2048
    rows = TWO31 // cols + 1
    x = normal(912, (PERIOD, cols), 4.0)
    x[3, ::5] = -np.inf
    small = dev_f32(x)
    backend.softmax_rows(small)
    assert_f32_close(host_f32(small), oracle.softmax_rows(x), 1e-5, "softmax_rows one period")
    big = tiled(dev_f32(x), rows)
    backend.softmax_rows(big)
    assert_periodic(big, small, f"softmax_rows f32 [{rows}, {cols}]")


def test_scale_mask_softmax_f32_past_2_31_elements(backend):
    batch, cols = 4, 1024
    rows = TWO31 // (batch * cols) + 1
    x = normal(913, (batch, PERIOD, cols), 4.0)
    mask = np.where(np.random.default_rng(914).uniform(size=(PERIOD, cols)) < 0.3, -np.inf, 0.0).astype(np.float32)
    small = dev_f32(x.reshape(batch * PERIOD, cols))
    backend.scale_mask_softmax_rows(small, 0.125, dev_f32(mask), batch, PERIOD, cols)
    want = oracle.softmax_rows(oracle.scale_add_mask(x.reshape(batch * PERIOD, cols), 0.125, mask, batch, PERIOD,
                                                     cols))
    assert_f32_close(host_f32(small), want, 1e-5, "scale_mask_softmax one period")
    big = torch.empty(batch, rows, cols, device="cuda")
    for s in range(batch):
        big[s].copy_(tiled(dev_f32(x[s]), rows))
    lmask = tiled(dev_f32(mask), rows)
    backend.scale_mask_softmax_rows(big.view(batch * rows, cols), 0.125, lmask, batch, rows, cols)
    for s in range(batch):
        assert_periodic(big[s], small.view(batch, PERIOD, cols)[s], f"scale_mask_softmax slice {s} [{rows}, {cols}]")


def test_gather_rows_past_2_31_output_elements(backend):
    vocab, cols = 1000, 2048
    rows = TWO31 // cols + 3
    table = oracle.f32_to_bf16(0.02 * normal(915, (vocab, cols)))
    ids = np.array([999, 0, 517, 3, 998, 250, 1], dtype=np.int64)
    out = torch.empty(rows, cols, device="cuda")
    backend.gather_rows_bf16(dev_bf16(table), tiled(dev_i64(ids).view(PERIOD, 1), rows).view(rows), out,
                             table_rows=vocab)
    assert_periodic(out, dev_f32(oracle.embed(table, ids)), f"gather_rows_bf16 [{rows}, {cols}]")


def test_copy_past_2_31_elements(backend):
    n = TWO31 + 5
    src = torch.empty(n, device="cuda").normal_(generator=torch.Generator("cuda").manual_seed(920))
    dst = torch.zeros_like(src)
    backend.copy(dst, src)
    assert torch.equal(bits(dst), bits(src)), f"copy n={n}"


@pytest.mark.parametrize("cache", ["f32", "bf16"])
def test_attend_step_past_2_31_cache_elements(backend, cache):
    heads, hd = 10, 128
    width = heads * hd
    capacity = TWO31 // width + 100
    live = np.array([0, 5, capacity // 2, TWO31 // width + 1, capacity - 2, capacity - 1], dtype=np.int64)
    dt = torch.float32 if cache == "f32" else torch.bfloat16
    kc = torch.zeros(capacity, width, dtype=dt, device="cuda")
    vc = torch.zeros(capacity, width, dtype=dt, device="cuda")
    kr, vr = normal(916, (len(live), width)), normal(917, (len(live), width))
    if cache == "bf16":
        kr, vr = oracle.bf16_round(kr), oracle.bf16_round(vr)
    idx = dev_i64(live)
    kc[idx] = dev_f32(kr).to(dt)
    vc[idx] = dev_f32(vr).to(dt)
    bias = normal(918, len(live), 0.5)
    mask = torch.full((capacity,), -np.inf, device="cuda")
    mask[idx] = dev_f32(bias)
    q = normal(919, width)
    state = dev_i64([0, capacity - 1, capacity - 1, 0, -1])
    scratch = torch.empty(backend.attend_scratch_floats(heads, hd, capacity), device="cuda")
    out = torch.empty(width, device="cuda")
    scale = float(1 / np.sqrt(hd))
    backend.attend_step(dev_f32(q), kc, vc, heads, hd, mask, scale, state, scratch, out)
    want = oracle.attention_one(q, kr, vr, heads, hd, bias=bias, scale=scale)
    assert_f32_close(host_f32(out), want, 1e-5, f"attend_step {cache} cache [{capacity}, {width}]")


# ---- launches in pieces: calls past a million rows run as several launches --------------------

PIECE_ROWS = 1 << 20  # rows per launch of the row kernels


# 4097 bf16 columns: the scalar path, 65 chunk groups, so the wide-row kernel
@pytest.mark.parametrize("op,cols", [("rms_f32", 12), ("add_rms_f32", 13), ("layer_bf16", 24), ("rms_bf16_wide", 4097)])
def test_norm_row_pieces(backend, op, cols):
    rows = PIECE_ROWS + 37
    bf = op.endswith("bf16") or op.endswith("wide")
    x = normal(930, (PERIOD, cols), 2.0, 0.3)
    d = normal(931, (PERIOD, cols))
    w, b = dev_f32(1 + 0.02 * normal(932, cols)), dev_f32(0.02 * normal(933, cols))
    up = (lambda a: dev_bf16(oracle.f32_to_bf16(a))) if bf else dev_f32
    small, sd = up(x), up(d)
    big, bd = tiled(small.clone(), rows), tiled(sd, rows)
    for t, dd in ((small, sd), (big, bd)):
        if op.startswith("rms"):
            backend.rms_norm(t, w, 1e-6)
        elif op.startswith("layer"):
            backend.layer_norm(t, w, b, 1e-6)
        else:
            h = torch.empty_like(t)
            backend.add_rms_norm(t, dd, w, h, 1e-6)
            if t is small:
                sh = h
            else:
                assert_periodic(h, sh, f"{op} h [{rows}, {cols}]")
    assert_periodic(big, small, f"{op} [{rows}, {cols}]")


def test_rope_row_pieces(backend):
    rows, dim = PIECE_ROWS + 3, 6  # half 3: the scalar path
    q, k = normal(934, (PERIOD, dim)), normal(935, (PERIOD, 2 * dim))
    tok, page = np.arange(PERIOD, dtype=np.int64) * 37, np.arange(PERIOD, dtype=np.int64) - 3
    inv_tok, inv_page = oracle.rope_inv(2, 1e4), oracle.rope_inv(1, 256.0)
    sq, sk = dev_f32(q), dev_f32(k)
    lq, lk = tiled(sq.clone(), rows), tiled(sk.clone(), rows)
    args = dict(inv_tok=dev_f32(inv_tok), inv_page=dev_f32(inv_page), page_mod=4)
    backend.rope_qk(sq, 1, sk, 2, dim, dev_i64(tok), dev_i64(page), **args)
    backend.rope_qk(lq, 1, lk, 2, dim, tiled(dev_i64(tok).view(PERIOD, 1), rows).view(rows),
                    tiled(dev_i64(page).view(PERIOD, 1), rows).view(rows), **args)
    assert_periodic(lq, sq, f"rope q [{rows}, 1 x {dim}]")
    assert_periodic(lk, sk, f"rope k [{rows}, 2 x {dim}]")


def test_softmax_row_pieces(backend):
    rows, cols = PIECE_ROWS + 9, 5
    x = normal(936, (PERIOD, cols), 3.0)
    small = dev_f32(x)
    big = tiled(small.clone(), rows)
    backend.softmax_rows(small)
    backend.softmax_rows(big)
    assert_periodic(big, small, f"softmax_rows [{rows}, {cols}]")
    batch, cols = 3, 7
    mrows = PIECE_ROWS // batch + 5
    x = normal(937, (batch, PERIOD, cols), 3.0)
    mask = np.where(np.random.default_rng(938).uniform(size=(PERIOD, cols)) < 0.3, -np.inf, 0.0).astype(np.float32)
    small = dev_f32(x.reshape(batch * PERIOD, cols))
    backend.scale_mask_softmax_rows(small, 0.5, dev_f32(mask), batch, PERIOD, cols)
    big = torch.empty(batch, mrows, cols, device="cuda")
    for s in range(batch):
        big[s].copy_(tiled(dev_f32(x[s]), mrows))
    backend.scale_mask_softmax_rows(big.view(batch * mrows, cols), 0.5, tiled(dev_f32(mask), mrows), batch, mrows,
                                    cols)
    for s in range(batch):
        assert_periodic(big[s], small.view(batch, PERIOD, cols)[s], f"scale_mask_softmax slice {s} [{mrows}, {cols}]")


def test_gather_row_pieces(backend):
    vocab, cols, rows = 50, 3, PIECE_ROWS + 11
    table = oracle.f32_to_bf16(normal(939, (vocab, cols)))
    ids = np.array([49, 0, 7, 60, 3, -1, 25], dtype=np.int64)  # 60 and -1 fall outside: zero rows
    out = torch.empty(rows, cols, device="cuda")
    backend.gather_rows_bf16(dev_bf16(table), tiled(dev_i64(ids).view(PERIOD, 1), rows).view(rows), out,
                             table_rows=vocab)
    want = oracle.embed(table, np.clip(ids, 0, vocab - 1))
    want[(ids < 0) | (ids >= vocab)] = 0.0
    assert_periodic(out, dev_f32(want), f"gather_rows_bf16 [{rows}, {cols}]")
