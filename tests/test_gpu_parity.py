"""GPU parity: every op through the C ABI against the CPU oracle, on the same
seeded inputs, at the tolerances in tests/parity.py. Small cases cover the
reference's own device test shapes (tests/cuda_ops_test.cpp:103-170) and the
edge cases (empty, ragged, misaligned, wide rows, page axis, out-of-range
ids); the config cases run the benchmark workloads at full size, where the
oracle still finishes in well under a second per op."""

import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from parity import (assert_bf16_close, assert_f32_close, dev_bf16, dev_f32, dev_i64, host_bits, host_f32,
                    normal)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def device(backend):
    if not torch.cuda.is_available() or backend.device_count() == 0:
        pytest.skip("no HIP device")
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


def weights(seed, cols):
    return (1 + 0.02 * normal(seed, cols)).astype(np.float32)


def bf16(a):
    return oracle.f32_to_bf16(a)


# ---- the reference's own device-test cases (fp32) ------------------------------------------------


def test_fp32_norms_and_activations(backend):
    x, w, b = normal(5, (9, 300)), normal(6, 300), normal(7, 300)
    d = dev_f32(x)
    backend.layer_norm(d, dev_f32(w), dev_f32(b), 1e-6)
    assert_f32_close(host_f32(d), oracle.layer_norm(x, w, b, 1e-6), 1e-5, "layer_norm")
    d = dev_f32(x)
    backend.rms_norm(d, dev_f32(w), 1e-6)
    assert_f32_close(host_f32(d), oracle.rms_norm(x, w, 1e-6), 1e-5, "rms_norm")
    d = dev_f32(x)
    backend.gelu_erf(d)
    assert_f32_close(host_f32(d), oracle.gelu_erf(x), 1e-6, "gelu_erf")
    u = normal(8, (9, 300))
    d = dev_f32(x)
    backend.silu_mul(d, dev_f32(u))
    assert_f32_close(host_f32(d), oracle.silu_mul(x, u), 1e-6, "silu_mul")
    d = dev_f32(x)
    backend.add_inplace(d, dev_f32(u))
    assert np.array_equal(host_f32(d), oracle.add(x, u))
    c = torch.empty_like(d)
    backend.copy(c, d)
    assert torch.equal(c, d)


def test_fp32_rope_page2d(backend):
    # tests/cuda_ops_test.cpp:142-162: PageRope(16), coordinates (0,0) (5,1) (300,2) (7,3)
    x = normal(9, (4, 32))
    tok, page = np.array([0, 5, 300, 7]), np.array([0, 1, 2, 3])
    inv_tok, inv_page = oracle.rope_inv(7, 1e4), np.array([1.0], np.float32)
    want = oracle.rope(x, 2, 16, tok=tok, page=page, inv_tok=inv_tok, inv_page=inv_page, page_mod=2)
    d = dev_f32(x)
    backend.rope(d, 2, 16, dev_i64(tok), dev_i64(page), dev_f32(inv_tok), dev_f32(inv_page), 2)
    assert_f32_close(host_f32(d), want, 1e-5, "rope page2d")


def test_fp32_fused_ops(backend):
    x, dl, w = normal(10, (37, 2048)), normal(11, (37, 2048)), weights(12, 2048)
    wx, wh = oracle.add_rms_norm(x, dl, w, 1e-6)
    dx, h = dev_f32(x), torch.empty(37, 2048, device="cuda")
    backend.add_rms_norm(dx, dev_f32(dl), dev_f32(w), h, 1e-6)
    assert np.array_equal(host_f32(dx), wx)  # the residual sum is one fp32 add
    assert_f32_close(host_f32(h), wh, 1e-5, "add_rms_norm")
    inp = normal(13, (21, 2 * 1408))
    out = torch.empty(21, 1408, device="cuda")
    backend.swiglu(dev_f32(inp), out)
    assert_f32_close(host_f32(out), oracle.swiglu(inp), 1e-6, "swiglu")
    q, k = normal(14, (5, 16 * 128)), normal(15, (5, 4 * 128))
    pos = np.array([0, 1, 999, 8191, 20000])
    inv = oracle.rope_inv(64, 1e4)
    dq, dk = dev_f32(q), dev_f32(k)
    backend.rope_qk(dq, 16, dk, 4, 128, dev_i64(pos), None, dev_f32(inv), None, 0)
    assert_f32_close(host_f32(dq), oracle.rope(q, 16, 128, tok=pos, inv_tok=inv), 1e-5, "rope_qk q")
    assert_f32_close(host_f32(dk), oracle.rope(k, 4, 128, tok=pos, inv_tok=inv), 1e-5, "rope_qk k")


# ---- gather: bit-exact -------------------------------------------------------------------------------


def test_gather_exact(backend):
    g = np.random.default_rng(16)
    table = g.integers(0, 1 << 16, (300, 2048), dtype=np.uint16)  # every bit pattern, NaNs included
    ids = np.array([299, 0, 17, 17, 150], np.int64)
    dt, di = dev_bf16(table), dev_i64(ids)
    out = torch.empty(5, 2048, device="cuda")
    backend.gather_rows_bf16(dt, di, out)
    assert np.array_equal(host_f32(out).view(np.uint32), oracle.embed(table, ids).view(np.uint32))
    outb = torch.empty(5, 2048, dtype=torch.bfloat16, device="cuda")
    backend.gather_rows_bf16(dt, di, outb)
    assert np.array_equal(host_bits(outb), table[ids])
    one = torch.empty(2048, device="cuda")
    backend.gather_row_bf16(dt, 123, one)
    assert np.array_equal(host_f32(one).view(np.uint32), oracle.embed(table, [123])[0].view(np.uint32))


def test_gather_out_of_range_ids_give_zero_rows(backend):
    table = np.random.default_rng(17).integers(0, 1 << 16, (64, 40), dtype=np.uint16)
    ids = np.array([3, -1, 64, 1 << 40, 63], np.int64)
    out = torch.full((5, 40), 7.0, device="cuda")
    backend.gather_rows_bf16(dev_bf16(table), dev_i64(ids), out)
    got = host_f32(out)
    assert np.all(got[1:4] == 0)
    assert np.array_equal(got[[0, 4]].view(np.uint32), oracle.embed(table, ids[[0, 4]]).view(np.uint32))


def test_gather_ragged_width_takes_scalar_path(backend):
    table = np.random.default_rng(18).integers(0, 1 << 16, (10, 13), dtype=np.uint16)
    ids = np.array([9, 2, 5], np.int64)
    out = torch.empty(3, 13, device="cuda")
    backend.gather_rows_bf16(dev_bf16(table), dev_i64(ids), out)
    assert np.array_equal(host_f32(out).view(np.uint32), oracle.embed(table, ids).view(np.uint32))


# ---- bf16 ops, small and edge cases ---------------------------------------------------------------------


@pytest.mark.parametrize("rows,cols", [(1, 2048), (5, 2048), (33, 1280), (7, 768), (6, 300), (3, 13),
                                       (2, 20000), (4, 8192), (0, 2048)])
def test_bf16_add_rms_norm_shapes(backend, rows, cols):
    x, dl, w = bf16(normal(rows + cols, (rows, cols))), bf16(normal(rows * 3 + 1, (rows, cols))), weights(cols, cols)
    wx, wh = oracle.add_rms_norm(oracle.bf16_to_f32(x), oracle.bf16_to_f32(dl), w, 1e-6)
    dx, h = dev_bf16(x), torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda")
    backend.add_rms_norm(dx, dev_bf16(dl), dev_f32(w), h, 1e-6)
    if rows == 0:
        return
    assert np.array_equal(host_bits(dx), bf16(wx))  # x' = bf16(x + delta) exactly
    assert_bf16_close(host_bits(h), wh, f"add_rms_norm_bf16 {rows}x{cols}")


@pytest.mark.parametrize("rows,cols", [(4, 1024), (9, 300), (3, 13), (2, 20000), (1, 3072)])
def test_bf16_layer_norm_and_gelu_shapes(backend, rows, cols):
    x = bf16(normal(cols, (rows, cols), 2.0, 0.5))
    w, b = weights(cols + 1, cols), (0.02 * normal(cols + 2, cols)).astype(np.float32)
    d = dev_bf16(x)
    backend.layer_norm(d, dev_f32(w), dev_f32(b), 1e-6)
    ln = host_bits(d)
    assert_bf16_close(ln, oracle.layer_norm(oracle.bf16_to_f32(x), w, b, 1e-6), f"layer_norm_bf16 {rows}x{cols}")
    backend.gelu_erf(d)
    assert_bf16_close(host_bits(d), oracle.gelu_erf(oracle.bf16_to_f32(ln)), f"gelu_erf_bf16 {rows}x{cols}")


@pytest.mark.parametrize("rows,ffn", [(1, 1408), (9, 1408), (5, 896), (3, 13), (2, 5000)])
def test_bf16_swiglu_shapes(backend, rows, ffn):
    inp = bf16(normal(ffn, (rows, 2 * ffn), 2.0))
    out = torch.empty(rows, ffn, dtype=torch.bfloat16, device="cuda")
    backend.swiglu(dev_bf16(inp), out)
    assert_bf16_close(host_bits(out), oracle.swiglu(oracle.bf16_to_f32(inp)), f"swiglu_bf16 {rows}x{ffn}")


# Elementwise grids switch from four-wave to one-wave workgroups past 655360
# threads (1.25 resident rounds of waves): sizes at, just past and well past
# that boundary, with ragged tails, for every flat op and dtype.
@pytest.mark.parametrize("chunks,tail", [(655360, 0), (655361, 3), (1 << 20, 7)])
def test_flat_ops_across_workgroup_size_switch(backend, chunks, tail):
    n = 8 * chunks + tail
    x = normal(chunks + tail, n, 2.0)
    xb = bf16(x)
    d = dev_bf16(xb)
    backend.gelu_erf(d)
    assert_bf16_close(host_bits(d), oracle.gelu_erf(oracle.bf16_to_f32(xb)), f"gelu_erf_bf16 n={n}")
    d = dev_bf16(xb)
    backend.quick_gelu(d)
    assert_bf16_close(host_bits(d), oracle.quick_gelu(oracle.bf16_to_f32(xb)), f"quick_gelu_bf16 n={n}")
    n32 = 4 * chunks + tail
    x32, y32 = x[:n32].copy(), normal(chunks + 1, n32)
    d = dev_f32(x32)
    backend.gelu_erf(d)
    assert_f32_close(host_f32(d), oracle.gelu_erf(x32), 1e-6, f"gelu_erf n={n32}")
    g, u = dev_f32(x32), dev_f32(y32)
    backend.silu_mul(g, u)
    assert_f32_close(host_f32(g), oracle.silu_mul(x32, y32), 1e-6, f"silu_mul n={n32}")
    a = dev_f32(x32)
    backend.add_inplace(a, dev_f32(y32))
    assert np.array_equal(host_f32(a), oracle.add(x32, y32)), f"add_inplace n={n32}"


@pytest.mark.parametrize("n,offset", [(1, 0), (3, 0), (4097, 0), (4099, 1), (2_097_152, 0), (2_097_163, 0),
                                      (2_621_440, 0), (2_621_447, 0), (4_194_304 + 7, 0), (1_000_003, 3),
                                      (600_001, 1)])
def test_copy_bitwise(backend, n, offset):
    """copy moves every bit (NaN payloads and signed zeros included) across
    the vector and scalar paths, ragged tails, the two-chunks-per-thread grids
    (just over one resident round) and the workgroup-size switch; `offset`
    elements past a 16-byte boundary takes the scalar path."""
    g = np.random.default_rng(n)
    bits = g.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    src = torch.empty(n + 8, device="cuda")
    dst = torch.full((n + 8,), 7.0, device="cuda")
    sv, dv = src[offset:offset + n], dst[offset:offset + n]
    sv.copy_(torch.from_numpy(bits.view(np.float32)).cuda())
    backend.copy(dv, sv)
    got = dst.cpu().numpy()
    assert np.array_equal(got[offset:offset + n].view(np.uint32), bits), f"copy n={n} offset={offset}"
    assert np.all(got[:offset] == 7.0) and np.all(got[offset + n:] == 7.0), "copy wrote outside dst"


@pytest.mark.parametrize("rows,ffn", [(3723, 1408), (3724, 1408), (50413, 13)])
def test_bf16_swiglu_across_workgroup_size_switch(backend, rows, ffn):
    inp = bf16(normal(rows + ffn, (rows, 2 * ffn), 2.0))
    out = torch.empty(rows, ffn, dtype=torch.bfloat16, device="cuda")
    backend.swiglu(dev_bf16(inp), out)
    assert_bf16_close(host_bits(out), oracle.swiglu(oracle.bf16_to_f32(inp)), f"swiglu_bf16 {rows}x{ffn}")


@pytest.mark.parametrize("dim,qh,kh,n_page", [(128, 16, 4, 0), (128, 10, 10, 1), (64, 1, 0, 0), (16, 2, 1, 1),
                                              (6, 3, 2, 0), (512, 2, 1, 0)])
def test_bf16_rope_shapes(backend, dim, qh, kh, n_page):
    rows, half = 19, dim // 2
    g = np.random.default_rng(dim + qh)
    q, k = bf16(normal(dim, (rows, qh * dim))), bf16(normal(dim + 1, (rows, max(kh, 1) * dim)))
    tok = g.integers(-30000, 30000, rows)
    page = g.integers(-9, 9, rows)
    inv_tok = oracle.rope_inv(half - n_page, 1e4)
    inv_page = oracle.rope_inv(n_page, 256.0) if n_page else None
    dq, dk = dev_bf16(q), dev_bf16(k)
    backend.rope_qk(dq, qh, dk if kh else None, kh, dim, dev_i64(tok), dev_i64(page), dev_f32(inv_tok),
                    dev_f32(inv_page) if n_page else None, 2)
    wq = oracle.rope(oracle.bf16_to_f32(q), qh, dim, tok=tok, page=page, inv_tok=inv_tok, inv_page=inv_page,
                     page_mod=2)
    assert_bf16_close(host_bits(dq), wq, f"rope_qk_bf16 q dim {dim}")
    if kh:
        wk = oracle.rope(oracle.bf16_to_f32(k), kh, dim, tok=tok, page=page, inv_tok=inv_tok, inv_page=inv_page,
                         page_mod=2)
        assert_bf16_close(host_bits(dk), wk, f"rope_qk_bf16 k dim {dim}")
    else:
        assert np.array_equal(host_bits(dk), k)


def test_misaligned_views_take_scalar_path(backend):
    """Tensors starting one element past a 16-byte boundary."""
    rows, cols = 6, 1024
    base = torch.empty(rows * cols + 8, dtype=torch.bfloat16, device="cuda")
    x = bf16(normal(40, (rows, cols)))
    view = base[1:1 + rows * cols].view(rows, cols)
    view.copy_(dev_bf16(x))
    w = weights(41, cols)
    backend.rms_norm(view, dev_f32(w), 1e-6)
    assert_bf16_close(host_bits(view), oracle.rms_norm(oracle.bf16_to_f32(x), w, 1e-6), "rms_norm misaligned")
    gbase = torch.empty(cols + 8, dtype=torch.bfloat16, device="cuda")
    gv = gbase[1:1 + cols]
    gv.copy_(dev_bf16(x[0]))
    backend.gelu_erf(gv)
    assert_bf16_close(host_bits(gv), oracle.gelu_erf(oracle.bf16_to_f32(x[0])), "gelu misaligned")


def test_bf16_gelu_every_input(backend):
    """Every finite bf16 value through gelu_erf_bf16, element by element:
    above -4.6 the oracle's fp32 GELU rounded to bf16, or its neighbour;
    from -5.5 to -4.6, where the reference's own 1 + erf(x / sqrt 2)
    cancels, the exact GELU (fp64) rounded to bf16, or its neighbour; below
    -5.5 x * 0, which is the reference's result below -5.5426 (between, the
    reference's is fp32 noise under 2e-7)."""
    from scipy.special import ndtr

    def ulps(a_bits, b_bits):
        a, b = a_bits.astype(np.int64), b_bits.astype(np.int64)
        oa = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
        ob = np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
        return np.abs(oa - ob)

    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = oracle.bf16_to_f32(bits)
    keep = np.isfinite(x)
    bits, x = bits[keep], x[keep]
    d = dev_bf16(bits)
    backend.gelu_erf(d)
    got = host_bits(d)
    ref = bf16(oracle.gelu_erf(x))
    exact = bf16((x.astype(np.float64) * ndtr(x.astype(np.float64))).astype(np.float32))
    hi, mid, lo = x > -4.6, (x <= -4.6) & (x >= -5.5), x < -5.5
    assert ulps(got[hi], ref[hi]).max() <= 1, "gelu_erf_bf16 above -4.6"
    assert ulps(got[mid], exact[mid]).max() <= 1, "gelu_erf_bf16 in [-5.5, -4.6]"
    assert np.all(got[lo] == 0x8000), "gelu_erf_bf16 below -5.5 is -0"
    far = x < -5.5426
    assert np.array_equal(got[far], ref[far]), "gelu_erf_bf16 below -5.5426"


def test_flat_ops_ragged_tail(backend):
    for n in [1, 7, 9, 1001, 4099]:
        x = bf16(normal(n, n, 3.0))
        d = dev_bf16(x)
        backend.gelu_erf(d)
        assert_bf16_close(host_bits(d), oracle.gelu_erf(oracle.bf16_to_f32(x)), f"gelu n={n}")
        xf, uf = normal(n + 1, n), normal(n + 2, n)
        df = dev_f32(xf)
        backend.silu_mul(df, dev_f32(uf))
        assert_f32_close(host_f32(df), oracle.silu_mul(xf, uf), 1e-6, f"silu_mul n={n}")


def test_results_are_deterministic(backend):
    x, dl, w = bf16(normal(50, (64, 2048))), bf16(normal(51, (64, 2048))), weights(52, 2048)
    outs = []
    for _ in range(2):
        dx, h = dev_bf16(x), torch.empty(64, 2048, dtype=torch.bfloat16, device="cuda")
        backend.add_rms_norm(dx, dev_bf16(dl), dev_f32(w), h, 1e-6)
        outs.append(host_bits(h))
    assert np.array_equal(outs[0], outs[1])


# ---- the benchmark workloads at full size ------------------------------------------------------------


def test_config1_fp32_rms_norm(backend):
    x, w = normal(0, (1024, 2048)), weights(1, 2048)
    d = dev_f32(x)
    backend.rms_norm(d, dev_f32(w), 1e-6)
    assert_f32_close(host_f32(d), oracle.rms_norm(x, w, 1e-6), 1e-5, "config 1 rms_norm")


def test_config2_decode_chain(backend):
    g = np.random.default_rng(2)
    vocab, hidden = 128000, 2048
    table = bf16(0.02 * g.standard_normal((vocab, hidden), dtype=np.float32))
    token = int(g.integers(0, vocab))
    pos = int(g.integers(0, 20001))
    dl, w = bf16(normal(3, hidden)), weights(4, hidden)
    q, k = bf16(normal(5, 16 * 128)), bf16(normal(6, 4 * 128))
    inv = oracle.rope_inv(64, 1e4)
    dt = dev_bf16(table)
    state = dev_i64([token, pos, pos, 0, -1])
    x = torch.empty(hidden, dtype=torch.bfloat16, device="cuda")
    h = torch.empty_like(x)
    dq, dk = dev_bf16(q), dev_bf16(k)
    backend.embed_step(dt, state, x)
    backend.add_rms_norm(x, dev_bf16(dl), dev_f32(w), h, 1e-6)
    backend.rope_qk_step(dq, 16, dk, 4, 128, state, dev_f32(inv), None, 0)
    e = oracle.embed(table, [token])[0]
    assert np.array_equal(host_bits(x), bf16(e + oracle.bf16_to_f32(dl)))
    _, wh = oracle.add_rms_norm(e, oracle.bf16_to_f32(dl), w, 1e-6)
    assert_bf16_close(host_bits(h), wh, "config 2 h")
    assert_bf16_close(host_bits(dq), oracle.rope(oracle.bf16_to_f32(q), 16, 128, inv_tok=inv, one_tok=pos), "q")
    assert_bf16_close(host_bits(dk), oracle.rope(oracle.bf16_to_f32(k), 4, 128, inv_tok=inv, one_tok=pos), "k")
    # the last row of the 500 MB table: byte offsets past 2^31
    last = torch.empty(hidden, device="cuda")
    backend.gather_row_bf16(dt, vocab - 1, last)
    assert np.array_equal(host_f32(last).view(np.uint32), oracle.embed(table, [vocab - 1])[0].view(np.uint32))


def test_config3_rope_prefill(backend):
    rows = 8192
    q, k = bf16(normal(30, (rows, 16 * 128))), bf16(normal(31, (rows, 4 * 128)))
    pos = np.arange(rows, dtype=np.int64)
    inv = oracle.rope_inv(64, 1e4)
    dq, dk = dev_bf16(q), dev_bf16(k)
    backend.rope_qk(dq, 16, dk, 4, 128, dev_i64(pos), None, dev_f32(inv), None, 0)
    assert_bf16_close(host_bits(dq), oracle.rope(oracle.bf16_to_f32(q), 16, 128, tok=pos, inv_tok=inv), "cfg3 q")
    assert_bf16_close(host_bits(dk), oracle.rope(oracle.bf16_to_f32(k), 4, 128, tok=pos, inv_tok=inv), "cfg3 k")


def test_config4_vision_layer_norm_gelu(backend):
    x = bf16(normal(40, (4096, 1024)))
    w, b = weights(41, 1024), (0.02 * normal(42, 1024)).astype(np.float32)
    d = dev_bf16(x)
    backend.layer_norm(d, dev_f32(w), dev_f32(b), 1e-6)
    ln = host_bits(d)
    assert_bf16_close(ln, oracle.layer_norm(oracle.bf16_to_f32(x), w, b, 1e-6), "cfg4 layer_norm")
    backend.gelu_erf(d)
    assert_bf16_close(host_bits(d), oracle.gelu_erf(oracle.bf16_to_f32(ln)), "cfg4 gelu")


def test_config5_prefill_chain(backend):
    rows, hidden, ffn = 8192, 2048, 1408
    x, dl, w = bf16(normal(50, (rows, hidden))), bf16(normal(51, (rows, hidden))), weights(52, hidden)
    inp = bf16(normal(53, (rows, 2 * ffn)))
    dx, h = dev_bf16(x), torch.empty(rows, hidden, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(rows, ffn, dtype=torch.bfloat16, device="cuda")
    backend.add_rms_norm(dx, dev_bf16(dl), dev_f32(w), h, 1e-6)
    backend.swiglu(dev_bf16(inp), out)
    wx, wh = oracle.add_rms_norm(oracle.bf16_to_f32(x), oracle.bf16_to_f32(dl), w, 1e-6)
    assert np.array_equal(host_bits(dx), bf16(wx))
    assert_bf16_close(host_bits(h), wh, "cfg5 add_rms_norm")
    assert_bf16_close(host_bits(out), oracle.swiglu(oracle.bf16_to_f32(inp)), "cfg5 swiglu")
    # property at full size: rms of h / w is 1 on every row (w, eps aside)
    hh = oracle.bf16_to_f32(host_bits(h)).astype(np.float64) / w
    rms = np.sqrt(np.mean(hh * hh, axis=1))
    assert np.all(np.abs(rms - 1) < 4e-3)


# ---- graphs and the C++ suite ------------------------------------------------------------------------


def test_decode_chain_graph_replays(backend):
    """Capture gather -> add+RMSNorm -> rope_qk on a side stream, replay it
    at several step states with eager work and synchronisations between
    replays, and check every replay."""
    g = np.random.default_rng(60)
    vocab, hidden = 4096, 2048
    table = bf16(0.02 * g.standard_normal((vocab, hidden), dtype=np.float32))
    w, inv = weights(61, hidden), oracle.rope_inv(64, 1e4)
    dt, dw, dinv = dev_bf16(table), dev_f32(w), dev_f32(inv)
    state = torch.zeros(5, dtype=torch.int64, device="cuda")
    x = torch.empty(hidden, dtype=torch.bfloat16, device="cuda")
    dl, h = torch.empty_like(x), torch.empty_like(x)
    q = torch.empty(16 * 128, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(4 * 128, dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        backend.embed_step(dt, state, x)
        backend.add_rms_norm(x, dl, dw, h, 1e-6)
        backend.rope_qk_step(q, 16, k, 4, 128, state, dinv, None, 0)
    for step in range(4):
        token, pos = int(g.integers(0, vocab)), int(g.integers(0, 20001))
        dv, qv, kv = bf16(normal(70 + step, hidden)), bf16(normal(80 + step, 2048)), bf16(normal(90 + step, 512))
        state.copy_(torch.tensor([token, pos, pos, 0, -1]))
        dl.copy_(dev_bf16(dv))
        q.copy_(dev_bf16(qv))
        k.copy_(dev_bf16(kv))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        e = oracle.embed(table, [token])[0]
        wx, wh = oracle.add_rms_norm(e, oracle.bf16_to_f32(dv), w, 1e-6)
        assert np.array_equal(host_bits(x), bf16(wx))
        assert_bf16_close(host_bits(h), wh, f"replay {step} h")
        assert_bf16_close(host_bits(q), oracle.rope(oracle.bf16_to_f32(qv), 16, 128, inv_tok=inv, one_tok=pos), "q")
        assert_bf16_close(host_bits(k), oracle.rope(oracle.bf16_to_f32(kv), 4, 128, inv_tok=inv, one_tok=pos), "k")


def test_cpp_rocm_ops_test(backend):
    """The plain-main C++ parity test over the uocr::rocm layer."""
    binary = os.path.join(os.path.dirname(backend.LIB_PATH), "rocm_ops_test")
    r = subprocess.run([binary], capture_output=True, text=True, timeout=120)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_rope_qk_with_k_below_q_in_memory(backend):
    """Q and K as views of one buffer with K first: the kernel must not
    assume any order between the two tensors."""
    rows, dim = 23, 128
    q, k = bf16(normal(70, (rows, 16 * dim))), bf16(normal(71, (rows, 4 * dim)))
    pos = np.arange(rows, dtype=np.int64) * 911
    inv = oracle.rope_inv(64, 1e4)
    buf = torch.empty(rows * 20 * dim, dtype=torch.bfloat16, device="cuda")
    dk, dq = buf[: rows * 4 * dim], buf[rows * 4 * dim:]
    dk.copy_(dev_bf16(k).view(-1))
    dq.copy_(dev_bf16(q).view(-1))
    backend.rope_qk(dq, 16, dk, 4, dim, dev_i64(pos), None, dev_f32(inv), None, 0)
    assert_bf16_close(host_bits(dq), oracle.rope(oracle.bf16_to_f32(q), 16, dim, tok=pos, inv_tok=inv), "q")
    assert_bf16_close(host_bits(dk), oracle.rope(oracle.bf16_to_f32(k), 4, dim, tok=pos, inv_tok=inv), "k")


@pytest.mark.parametrize("mode", ["rms", "add_rms", "layer"])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_norm_rows_are_batch_invariant(backend, mode, dtype):
    """A row's norm is bitwise the same whether it is normalised alone (the
    kernel spreads a row over 4 waves) or in a 3000-row batch (one wave per
    row): the reduction order depends only on cols."""
    cols, rows = 2048, 3000
    x, dl = normal(80, (rows, cols)), normal(81, (rows, cols))
    w, b = weights(82, cols), (0.02 * normal(83, cols)).astype(np.float32)
    if dtype == "bf16":
        x, dl = oracle.bf16_round(x), oracle.bf16_round(dl)
        dev = lambda a: dev_bf16(oracle.f32_to_bf16(a))  # noqa: E731
        back = lambda t: oracle.bf16_to_f32(host_bits(t))  # noqa: E731
    else:
        dev, back = dev_f32, host_f32

    def run(sl):
        dx, dd = dev(x[sl]), dev(dl[sl])
        h = torch.empty_like(dx)
        if mode == "rms":
            backend.rms_norm(dx, dev_f32(w), 1e-6)
            return back(dx)
        if mode == "layer":
            backend.layer_norm(dx, dev_f32(w), dev_f32(b), 1e-6)
            return back(dx)
        backend.add_rms_norm(dx, dd, dev_f32(w), h, 1e-6)
        return back(h)

    full = run(slice(0, rows))
    for r in (0, 1234, rows - 1):
        alone = run(slice(r, r + 1))
        assert np.array_equal(alone.view(np.uint32), full[r:r + 1].view(np.uint32)), (mode, dtype, r)
