"""GPU parity for the ops on either side of the fused chain: the router norm,
quick GELU, softmax_rows and scale_add_mask (prefill and vision attention),
the bf16 weight-streaming GEMV and the decode step's append_step and
attend_step. Each runs through the C ABI on seeded inputs and is checked
against the CPU oracle at the tolerances of tests/parity.py; edge cases
follow the reference's own tests of these ops (tests/cuda_ops_test.cpp,
tests/cuda_decode_step_test.cpp): ragged and misaligned widths, masked and
fully masked rows, positions at and past the cache capacity."""

import numpy as np
import pytest

import oracle
from parity import assert_bf16_close, assert_f32_close, dev_bf16, dev_f32, dev_i64, host_bits, host_f32, normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def device(backend):
    if not torch.cuda.is_available() or backend.device_count() == 0:
        pytest.skip("no HIP device")
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


def bf16(a):
    return oracle.f32_to_bf16(a)


def state_of(pos, token=0):
    return dev_i64([token, pos, pos, 0, -1])


# ---- router norm, quick GELU ------------------------------------------------------------------


@pytest.mark.parametrize("rows,cols", [(1, 128), (9, 300), (37, 2048), (4096, 64), (3, 20000)])
def test_router_norm(backend, rows, cols):
    x = normal(100 + rows, (rows, cols))
    x[0, :3] = [np.nan, np.inf, -np.inf]  # zeroed before the sum
    w = (0.02 * normal(101, cols)).astype(np.float32)
    w[::7] = 2e4  # (1 + w) * n leaves the clamp range
    want = oracle.router_norm(x, w, 1e-6)
    d = dev_f32(x)
    backend.router_norm(d, dev_f32(w), 1e-6)
    got = host_f32(d)
    assert np.all(np.isfinite(got)) and np.max(np.abs(got)) <= 1e4
    assert_f32_close(got, want, 1e-5, "router_norm")
    xb = bf16(x)
    db = dev_bf16(xb)
    backend.router_norm(db, dev_f32(w), 1e-6)
    assert_bf16_close(host_bits(db), oracle.router_norm(oracle.bf16_to_f32(xb), w, 1e-6), "router_norm bf16")


@pytest.mark.parametrize("n", [1, 7, 4096, 1 << 20])
def test_quick_gelu(backend, n):
    x = 4 * normal(110, n)
    d = dev_f32(x)
    backend.quick_gelu(d)
    assert_f32_close(host_f32(d), oracle.quick_gelu(x), 1e-6, "quick_gelu")
    xb = bf16(x)
    db = dev_bf16(xb)
    backend.quick_gelu(db)
    assert_bf16_close(host_bits(db), oracle.quick_gelu(oracle.bf16_to_f32(xb)), "quick_gelu bf16")


# ---- softmax_rows, scale_add_mask ---------------------------------------------------------------


@pytest.mark.parametrize("rows,cols", [(1, 1), (9, 300), (64, 1024), (4096, 256), (2, 8192), (3, 20000),
                                       (5, 20003)])
def test_softmax_rows(backend, rows, cols):
    x = 3 * normal(120 + cols, (rows, cols))
    g = np.random.default_rng(121)
    x[g.random((rows, cols)) < 0.3] = -np.inf  # masked entries
    if rows > 1:
        x[1, :] = -np.inf  # a fully masked row becomes zeros
    want = oracle.softmax_rows(x)
    d = dev_f32(x)
    backend.softmax_rows(d)
    got = host_f32(d)
    assert_f32_close(got, want, 1e-5, "softmax_rows")
    if rows > 1:
        assert np.all(got[1] == 0)
    live = np.any(np.isfinite(x), axis=1)
    assert np.allclose(got[live].sum(axis=1, dtype=np.float64), 1.0, atol=1e-5)


def test_softmax_rows_are_batch_invariant(backend):
    cols = 1024
    x = normal(130, (4096, cols))
    one = dev_f32(x[:1])
    many = dev_f32(x)
    backend.softmax_rows(one)
    backend.softmax_rows(many)
    assert np.array_equal(host_f32(one)[0], host_f32(many)[0])


@pytest.mark.parametrize("batch,rows,cols,masked", [(16, 33, 47, True), (8, 64, 64, True), (10, 577, 577, True),
                                                    (4, 16, 16, False), (33, 8, 12, True), (1, 7, 9, False),
                                                    (3, 256, 256, True)])
def test_scale_add_mask(backend, batch, rows, cols, masked):
    x = normal(140, (batch, rows, cols))
    mask = None
    if masked:
        mask = np.triu(np.full((rows, cols), -np.inf, np.float32), 1)  # causal
        mask += 0.1 * normal(141, (rows, cols))
    want = oracle.scale_add_mask(x, 0.125, mask, batch, rows, cols)
    d = dev_f32(x)
    backend.scale_add_mask(d, 0.125, None if mask is None else dev_f32(mask), batch, rows, cols)
    assert np.array_equal(host_f32(d), want)


@pytest.mark.parametrize("batch,rows,cols,masked", [(10, 577, 577, True), (16, 64, 1024, True), (3, 33, 47, False),
                                                    (2, 5, 20000, True), (4, 4096, 256, True)])
def test_scale_mask_softmax_matches_the_pair(backend, batch, rows, cols, masked):
    x = 4 * normal(145, (batch, rows, cols))
    mask = None
    if masked:
        mask = np.triu(np.full((rows, cols), -np.inf, np.float32), 1) + 0.1 * normal(146, (rows, cols))
        mask[1 % rows, :] = -np.inf  # a fully masked row becomes zeros
    dm = None if mask is None else dev_f32(mask)
    pair, fused = dev_f32(x), dev_f32(x)
    backend.scale_add_mask(pair, 0.088, dm, batch, rows, cols)
    backend.softmax_rows(pair.view(batch * rows, cols))
    backend.scale_mask_softmax_rows(fused, 0.088, dm, batch, rows, cols)
    assert np.array_equal(host_f32(fused).view(np.uint32), host_f32(pair).view(np.uint32))
    want = oracle.softmax_rows(oracle.scale_add_mask(x, 0.088, mask, batch, rows, cols).reshape(-1, cols))
    assert_f32_close(host_f32(fused).reshape(-1, cols), want, 1e-5, "scale_mask_softmax")


# ---- GEMV ---------------------------------------------------------------------------------------


@pytest.mark.parametrize("k,n,with_bias", [(1280, 1280, True), (1280, 3840, False), (896, 1280, False),
                                           (2048, 20000, True), (4096, 300, True), (12288, 64, False),
                                           (100, 33, True), (8, 5, False),
                                           # more row pairs than the grid's waves: grid-stride rows
                                           (1280, 60001, True)])
def test_gemv_bf16(backend, k, n, with_bias):
    x = normal(150 + k, k)
    wb = bf16(0.05 * normal(151, (n, k)))
    bias = normal(152, n) if with_bias else None
    want = oracle.linear(oracle.bf16_round(x), oracle.bf16_to_f32(wb), bias)[0]
    y = torch.empty(n, device="cuda")
    backend.gemv_bf16(dev_f32(x), dev_bf16(wb), y, None if bias is None else dev_f32(bias))
    assert_f32_close(host_f32(y), want, 1e-5, f"gemv k={k} n={n}")


def test_gemv_bf16_misaligned_input_and_empty_k(backend):
    k, n = 1280, 96
    x = normal(160, k + 1)
    wb = bf16(0.05 * normal(161, (n, k)))
    dx = dev_f32(x)[1:]  # 4-byte offset: the element-wise kernel
    y = torch.empty(n, device="cuda")
    backend.gemv_bf16(dx, dev_bf16(wb), y)
    want = oracle.linear(oracle.bf16_round(x[1:]), oracle.bf16_to_f32(wb))[0]
    assert_f32_close(host_f32(y), want, 1e-5, "gemv misaligned")
    bias = normal(162, n)
    backend.gemv_bf16(torch.empty(0, device="cuda"), torch.empty(n, 0, dtype=torch.bfloat16, device="cuda"), y,
                      dev_f32(bias))
    assert np.array_equal(host_f32(y), bias)


# ---- append_step, attend_step -------------------------------------------------------------------


@pytest.mark.parametrize("width", [1280, 1283])
def test_append_step(backend, width):
    cap = 16
    cache = torch.zeros(cap, width, device="cuda")
    row = normal(170, width)
    drow = dev_f32(row)
    want = np.zeros((cap, width), np.float32)
    for pos in (0, 5, cap - 1):
        backend.append_step(cache, drow, state_of(pos))
        want[pos] = row
    for pos in (cap, cap + 3, -1):  # outside the cache: nothing is written
        backend.append_step(cache, drow, state_of(pos))
    assert np.array_equal(host_f32(cache), want)


def attend_case(backend, heads, hd, cap, pos, mask=None, scale=None, seed=0):
    width = heads * hd
    q = normal(seed, width)
    k = normal(seed + 1, (cap, width))
    v = normal(seed + 2, (cap, width))
    scale = 1.0 / np.sqrt(hd) if scale is None else scale
    keys = max(0, min(pos + 1, cap))
    want = oracle.attention_one(q, k[:keys], v[:keys], heads, hd, None if mask is None else mask[:keys], scale)
    scratch = torch.empty(max(1, backend.attend_scratch_floats(heads, hd, cap)), device="cuda")
    out = torch.full((width,), float("nan"), device="cuda")
    backend.attend_step(dev_f32(q), dev_f32(k), dev_f32(v), heads, hd, None if mask is None else dev_f32(mask),
                        float(scale), state_of(pos), scratch, out)
    return host_f32(out), want


@pytest.mark.parametrize("heads,hd,cap,pos", [(10, 128, 8192, 8191), (10, 128, 8192, 0), (10, 128, 8192, 100),
                                              (10, 128, 4096, 2999), (16, 64, 1024, 777), (4, 80, 500, 499),
                                              (2, 66, 300, 250), (2, 256, 700, 650), (3, 4, 100, 60),
                                              (1, 128, 7, 50), (10, 128, 64, 63),
                                              # past 8192 positions: four keys per batch, 16 lanes per key
                                              (10, 128, 16384, 12000), (4, 64, 9000, 8999), (2, 256, 9000, 5000),
                                              (3, 80, 10000, 9999)])
def test_attend_step(backend, heads, hd, cap, pos):
    got, want = attend_case(backend, heads, hd, cap, pos, seed=200 + hd)
    assert_f32_close(got, want, 1e-5, f"attend heads={heads} hd={hd} pos={pos}")


def test_attend_step_masked_blocks_and_all_masked(backend):
    heads, hd, cap = 10, 128, 4096
    mask = np.zeros(cap, np.float32)
    blocks = np.random.default_rng(210).random(cap // 64) < 0.6
    mask[np.repeat(blocks, 64)] = -np.inf  # routed blocks
    mask[3000] = 0.0
    mask[:64] += 0.25 * normal(211, 64)  # a finite bias on the first block
    got, want = attend_case(backend, heads, hd, cap, 3000, mask=mask, seed=212)
    assert_f32_close(got, want, 1e-5, "attend routed mask")
    none = np.full(cap, -np.inf, np.float32)
    got, _ = attend_case(backend, heads, hd, cap, 2000, mask=none, seed=213)
    assert np.array_equal(got, np.zeros_like(got))


def test_decode_attention_graph_replays(backend):
    """Capture append K, append V, attend on a side stream once; replay it at
    growing positions with eager work and synchronisations between replays,
    checking each replay against the oracle over the keys so far."""
    heads, hd, cap = 10, 128, 512
    width = heads * hd
    kc = torch.zeros(cap, width, device="cuda")
    vc = torch.zeros(cap, width, device="cuda")
    q, kr, vr = (torch.empty(width, device="cuda") for _ in range(3))
    out = torch.empty(width, device="cuda")
    scratch = torch.empty(backend.attend_scratch_floats(heads, hd, cap), device="cuda")
    state = torch.zeros(5, dtype=torch.int64, device="cuda")
    scale = 1.0 / np.sqrt(hd)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        backend.append_step(kc, kr, state)
        backend.append_step(vc, vr, state)
        backend.attend_step(q, kc, vc, heads, hd, None, scale, state, scratch, out)
    hk = np.zeros((cap, width), np.float32)
    hv = np.zeros((cap, width), np.float32)
    for pos in range(0, 300, 37):
        for p in range(int(state[1].item()) + 1 if pos else 0, pos):  # fill the gap eagerly
            hk[p], hv[p] = normal(1000 + p, width), normal(2000 + p, width)
            kc[p].copy_(dev_f32(hk[p]))
            vc[p].copy_(dev_f32(hv[p]))
        hk[pos], hv[pos] = normal(1000 + pos, width), normal(2000 + pos, width)
        qv = normal(3000 + pos, width)
        kr.copy_(dev_f32(hk[pos]))
        vr.copy_(dev_f32(hv[pos]))
        q.copy_(dev_f32(qv))
        state.copy_(torch.tensor([0, pos, pos, 0, -1]))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = oracle.attention_one(qv, hk[:pos + 1], hv[:pos + 1], heads, hd, None, scale)
        assert_f32_close(host_f32(out), want, 1e-5, f"replay pos={pos}")
        assert np.array_equal(host_f32(kc)[pos], hk[pos])


# ---- a bf16 key/value cache -----------------------------------------------------------------------


def host_bf16_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("width", [1280, 1283])
def test_append_step_bf16_rounds_the_row(backend, width):
    cap = 8
    cache = torch.zeros(cap, width, dtype=torch.bfloat16, device="cuda")
    row = normal(180, width)
    backend.append_step(cache, dev_f32(row), state_of(3))
    backend.append_step(cache, dev_f32(row), state_of(cap))  # past the cache: nothing
    got = host_bf16_bits(cache)
    assert np.array_equal(got[3], oracle.f32_to_bf16(row))
    assert not got[np.arange(cap) != 3].any()


@pytest.mark.parametrize("heads,hd,cap,pos", [(10, 128, 8192, 8191), (10, 128, 8192, 100), (16, 64, 1024, 777),
                                              (4, 80, 500, 499), (2, 66, 300, 250), (2, 256, 700, 650),
                                              (10, 128, 16384, 12000), (1, 128, 7, 50)])
def test_attend_step_bf16_cache(backend, heads, hd, cap, pos):
    width = heads * hd
    q = normal(190 + hd, width)
    kb, vb = bf16(normal(191, (cap, width))), bf16(normal(192, (cap, width)))
    scale = 1.0 / np.sqrt(hd)
    keys = max(0, min(pos + 1, cap))
    want = oracle.attention_one(q, oracle.bf16_to_f32(kb)[:keys], oracle.bf16_to_f32(vb)[:keys], heads, hd, None,
                                scale)
    scratch = torch.empty(max(1, backend.attend_scratch_floats(heads, hd, cap)), device="cuda")
    out = torch.full((width,), float("nan"), device="cuda")
    backend.attend_step(dev_f32(q), dev_bf16(kb), dev_bf16(vb), heads, hd, None, float(scale), state_of(pos), scratch,
                        out)
    assert_f32_close(host_f32(out), want, 1e-5, f"attend bf16 cache heads={heads} hd={hd} pos={pos}")


def test_attend_dead_keys_never_poison_the_sum(backend):
    """Masked and past-the-end keys load filler bits that the kernel must
    never multiply into the value sum: here every query float's low half is
    a bf16 NaN pattern, which a bf16 cache kernel reads as the filler."""
    heads, hd, cap, pos = 4, 128, 1024, 700
    width = heads * hd
    g = np.random.default_rng(195)
    hi = (g.integers(0x3C00, 0x4000, width, dtype=np.uint32) | (g.integers(0, 2, width, dtype=np.uint32) << 15))
    q = ((hi << 16) | np.uint32(0x7FC0)).view(np.float32)  # finite fp32, NaN low half
    assert np.all(np.isfinite(q)) and np.all(np.isnan(oracle.bf16_to_f32(np.full(1, 0x7FC0, np.uint16))))
    kb, vb = bf16(normal(196, (cap, width))), bf16(normal(197, (cap, width)))
    mask = np.where(g.random(cap) < 0.5, -np.inf, 0).astype(np.float32)
    mask[pos] = 0.0
    keys = pos + 1
    scale = 1.0 / np.sqrt(hd)
    want = oracle.attention_one(q, oracle.bf16_to_f32(kb)[:keys], oracle.bf16_to_f32(vb)[:keys], heads, hd,
                                mask[:keys], scale)
    scratch = torch.empty(backend.attend_scratch_floats(heads, hd, cap), device="cuda")
    for kc, vc in ((dev_bf16(kb), dev_bf16(vb)), (dev_f32(oracle.bf16_to_f32(kb)), dev_f32(oracle.bf16_to_f32(vb)))):
        out = torch.empty(width, device="cuda")
        backend.attend_step(dev_f32(q), kc, vc, heads, hd, dev_f32(mask), float(scale), state_of(pos), scratch, out)
        got = host_f32(out)
        assert np.all(np.isfinite(got))
        assert_f32_close(got, want, 1e-5, f"dead keys, {kc.dtype} cache")
