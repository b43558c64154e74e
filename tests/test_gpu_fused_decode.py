"""GPU parity for the fused decode-step ops. Each must give bitwise what the
unfused entry points give on the same inputs (that chain is itself checked
against the oracle in tests/test_gpu_step_ops.py and test_gpu_parity.py),
and is checked against the oracle directly as well:

  embed_add_rms_norm_step        == embed_step -> add_rms_norm (or copy -> rms_norm)
  add_rms_norm_gemv_bf16         == add_rms_norm (or rms_norm) -> gemv_bf16
  add_rms_norm_swiglu_gemv_bf16  == add_rms_norm -> gemv gate, gemv up -> silu_mul
  attend_rope_kv_step            == rope_qk_step -> append_step x2 -> attend_step
  attend_rope_kv_step_segments   == attend_rope_kv_step under the mask the
                                    segments describe (the same caches
                                    bitwise, the output within 1e-5: its
                                    splits sum in another order)
  attend_merge_gemv_bf16         == attend_rope_kv_step_segments' merge -> gemv_bf16

and a whole decode layer built from them replays in a graph bitwise like the
layer built from the unfused ops (the reference's decode_body order,
src/model/cuda/cuda_decode_step.cpp:47-66)."""

import numpy as np
import pytest

import oracle
from parity import (assert_bf16_close, assert_f32_close, dev_bf16, dev_f32, dev_i64, host_f32, key_segments,
                    mask_from_segments, normal)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def device(backend):
    if not torch.cuda.is_available() or backend.device_count() == 0:
        pytest.skip("no HIP device")
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


def bits(t):
    return host_f32(t).view(np.uint32)


def weights_bf16(seed, shape, scale=0.05):
    return dev_bf16(oracle.f32_to_bf16(scale * normal(seed, shape)))


def unfused_h(backend, x, delta, w_norm, eps=1e-6):
    """(x + delta, h) through the unfused ops, as the reference's decode step
    forms them (add_inplace + copy + rms_norm)."""
    k = x.numel()
    if delta is not None and w_norm is not None:
        xo, h = x.clone().view(1, k), torch.empty(1, k, device="cuda")
        backend.add_rms_norm(xo, delta.view(1, k), w_norm, h, eps)
        return xo.view(-1), h.view(-1)
    s = x.clone()
    if delta is not None:
        backend.add_inplace(s, delta)
    if w_norm is None:
        return s, s.clone()
    h = s.clone().view(1, k)
    backend.rms_norm(h, w_norm, eps)
    return s, h.view(-1)


@pytest.mark.parametrize("k,n,with_delta,with_norm,with_bias", [
    (1280, 3840, True, True, False), (1280, 1280, False, True, True), (2048, 2048, True, True, True),
    (896, 1280, True, False, False), (1280, 16384, True, True, False), (8, 5, False, False, True),
    (2048, 20000, True, True, True), (1024, 77, False, True, False),
    # more row pairs than the grid's waves: waves walk the rows grid-stride
    (256, 60001, True, True, True)])
def test_add_rms_norm_gemv_matches_unfused(backend, k, n, with_delta, with_norm, with_bias):
    x = dev_f32(normal(300 + k, k))
    delta = dev_f32(normal(301, k)) if with_delta else None
    w_norm = dev_f32(1 + 0.02 * normal(302, k)) if with_norm else None
    w = weights_bf16(303, (n, k))
    bias = dev_f32(normal(304, n)) if with_bias else None
    xu, hu = unfused_h(backend, x, delta, w_norm)
    yu = torch.empty(n, device="cuda")
    backend.gemv_bf16(hu, w, yu, bias)
    y, x_out, h_out = torch.empty(n, device="cuda"), torch.empty(k, device="cuda"), torch.empty(k, device="cuda")
    backend.add_rms_norm_gemv_bf16(x, w, y, delta=delta, x_out=x_out, w_norm=w_norm, h_out=h_out, bias=bias)
    assert np.array_equal(bits(y), bits(yu))
    assert np.array_equal(bits(h_out), bits(hu))
    assert np.array_equal(bits(x_out), bits(xu))
    # and against the oracle: h at the fp32 bar, y on the h it consumed
    hx = host_f32(x) + (host_f32(delta) if with_delta else 0)
    if with_norm:
        assert_f32_close(host_f32(h_out), oracle.rms_norm(hx[None], host_f32(w_norm), 1e-6)[0], 1e-5, "h")
    want = oracle.linear(oracle.bf16_round(host_f32(h_out)), oracle.bf16_to_f32(
        w.view(torch.int16).cpu().numpy().view(np.uint16)), None if bias is None else host_f32(bias))[0]
    assert_f32_close(host_f32(y), want, 1e-5, "y")


@pytest.mark.parametrize("k,ffn,with_delta", [(1280, 896, True), (2048, 1408, True), (1280, 896, False),
                                              (512, 20000, True)])
def test_add_rms_norm_swiglu_gemv_matches_unfused(backend, k, ffn, with_delta):
    x = dev_f32(normal(310, k))
    delta = dev_f32(normal(311, k)) if with_delta else None
    w_norm = dev_f32(1 + 0.02 * normal(312, k))
    wg, wu = weights_bf16(313, (ffn, k)), weights_bf16(314, (ffn, k))
    _, hu = unfused_h(backend, x, delta, w_norm)
    g, u = torch.empty(ffn, device="cuda"), torch.empty(ffn, device="cuda")
    backend.gemv_bf16(hu, wg, g)
    backend.gemv_bf16(hu, wu, u)
    backend.silu_mul(g, u)
    act = torch.empty(ffn, device="cuda")
    backend.add_rms_norm_swiglu_gemv_bf16(x, wg, wu, act, delta=delta, w_norm=w_norm)
    assert np.array_equal(bits(act), bits(g))
    hb = oracle.bf16_round(host_f32(hu))
    to_f = lambda t: oracle.bf16_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))  # noqa: E731
    want = oracle.silu_mul(oracle.linear(hb, to_f(wg))[0], oracle.linear(hb, to_f(wu))[0])
    assert_f32_close(host_f32(act), want, 1e-5, "swiglu gemv")


def test_fused_gemv_rejects_bad_arguments(backend):
    k, n = 1280, 16
    x, w, y = torch.randn(k, device="cuda"), weights_bf16(320, (n, k)), torch.empty(n, device="cuda")
    with pytest.raises(ValueError):  # x_out overlapping x: other workgroups still read it
        backend.add_rms_norm_gemv_bf16(x, w, y, x_out=x)
    with pytest.raises(ValueError):
        backend.add_rms_norm_gemv_bf16(torch.randn(4096, device="cuda"), weights_bf16(321, (n, 4096)), y)
    with pytest.raises(ValueError):
        backend.add_rms_norm_gemv_bf16(torch.randn(100, device="cuda"), weights_bf16(322, (n, 100)), y)
    with pytest.raises(ValueError):  # misaligned input row
        backend.add_rms_norm_gemv_bf16(torch.randn(k + 1, device="cuda")[1:], w, y)


def state_of(pos, tok=None, page=0):
    return dev_i64([0, pos, pos if tok is None else tok, page, -1])


@pytest.mark.parametrize("heads,hd,cap,pos,n_tok,page_mod,masked", [
    (10, 128, 8192, 5000, 64, 0, False), (10, 128, 8192, 8191, 48, 4, True), (4, 64, 300, 299, 32, 0, False),
    (2, 66, 100, 57, 33, 0, False), (2, 256, 9000, 8000, 100, 3, False), (10, 128, 64, 70, 64, 0, False),
    (3, 128, 512, 0, 64, 0, False), (10, 128, 2048, 1500, 64, 0, True), (4, 64, 300, 123, 0, 5, False)])
def test_attend_rope_kv_matches_unfused(backend, heads, hd, cap, pos, n_tok, page_mod, masked):
    width = heads * hd
    q, k_row, v_row = dev_f32(normal(330, width)), dev_f32(normal(331, width)), dev_f32(normal(332, width))
    kc0, vc0 = normal(333, (cap, width)), normal(334, (cap, width))
    half = hd // 2
    inv_tok = dev_f32(oracle.rope_inv(n_tok, 1e4)) if n_tok else None
    inv_page = dev_f32(oracle.rope_inv(half - n_tok, 100.0)) if n_tok < half else None
    mask = None
    if masked:
        m = np.where(np.random.default_rng(335).random(cap) < 0.4, -np.inf, 0).astype(np.float32)
        m[min(pos, cap - 1)] = -np.inf if pos % 2 else 0.0  # the step's own key masked or not
        mask = dev_f32(m)
    state = state_of(pos, tok=pos, page=pos // 7)
    scale = float(1 / np.sqrt(hd))
    scratch = torch.empty(backend.attend_scratch_floats(heads, hd, cap), device="cuda")
    # unfused chain
    qq, kk = q.clone(), k_row.clone()
    kc1, vc1 = dev_f32(kc0), dev_f32(vc0)
    out1 = torch.empty(width, device="cuda")
    backend.rope_qk_step(qq, heads, kk, heads, hd, state, inv_tok, inv_page, page_mod)
    backend.append_step(kc1, kk, state)
    backend.append_step(vc1, v_row, state)
    backend.attend_step(qq, kc1, vc1, heads, hd, mask, scale, state, scratch, out1)
    # fused
    kc2, vc2 = dev_f32(kc0), dev_f32(vc0)
    out2 = torch.empty(width, device="cuda")
    q_before, k_before = bits(q), bits(k_row)
    backend.attend_rope_kv_step(q, k_row, v_row, kc2, vc2, heads, hd, mask, scale, state, inv_tok, inv_page,
                                page_mod, scratch, out2)
    assert np.array_equal(bits(out2), bits(out1))
    assert np.array_equal(bits(kc2), bits(kc1)) and np.array_equal(bits(vc2), bits(vc1))
    assert np.array_equal(bits(q), q_before) and np.array_equal(bits(k_row), k_before)
    # against the oracle: rope the query, attend over the appended cache
    keys = max(0, min(pos + 1, cap))
    rq = oracle.rope(host_f32(q), heads, hd, inv_tok=None if inv_tok is None else host_f32(inv_tok),
                     inv_page=None if inv_page is None else host_f32(inv_page), page_mod=page_mod, one_tok=pos,
                     one_page=pos // 7)
    want = oracle.attention_one(rq, host_f32(kc2)[:keys], host_f32(vc2)[:keys], heads, hd,
                                None if mask is None else host_f32(mask)[:keys], scale)
    assert_f32_close(host_f32(out2), want, 1e-5, "attend_rope_kv")


def test_fused_decode_layer_graph_matches_unfused(backend):
    """One decoder layer's decode step, 11 unfused launches against 6 fused
    ones, each captured once and replayed at growing positions with eager
    work between replays; every replay's outputs must agree bitwise."""
    hidden, heads, hd, ffn, cap = 1280, 10, 128, 896, 512
    width = heads * hd
    inv = dev_f32(oracle.rope_inv(hd // 2, 1e4))
    scale = float(1 / np.sqrt(hd))
    wq, wk, wv = (weights_bf16(340 + i, (width, hidden), 0.03) for i in range(3))
    wqkv = torch.cat([wq, wk, wv]).contiguous()
    wo = weights_bf16(343, (hidden, width), 0.03)
    wg, wu = weights_bf16(344, (ffn, hidden), 0.03), weights_bf16(345, (ffn, hidden), 0.03)
    wd = weights_bf16(346, (hidden, ffn), 0.03)
    n1, n2 = dev_f32(1 + 0.02 * normal(347, hidden)), dev_f32(1 + 0.02 * normal(348, hidden))

    def buffers():
        b = {name: torch.zeros(size, device="cuda") for name, size in [
            ("x", hidden), ("delta", hidden), ("x1", hidden), ("x2", hidden), ("h", hidden), ("qkv", 3 * width),
            ("attn", width), ("o", hidden), ("g", ffn), ("u", ffn), ("act", ffn), ("out", hidden)]}
        b["kc"], b["vc"] = torch.zeros(cap, width, device="cuda"), torch.zeros(cap, width, device="cuda")
        b["scratch"] = torch.empty(backend.attend_scratch_floats(heads, hd, cap), device="cuda")
        b["state"] = torch.zeros(5, dtype=torch.int64, device="cuda")
        return b

    A, B = buffers(), buffers()

    def unfused(b):  # x1 = x + delta; h = norm(x1); qkv; rope; append; attend; o; x2 = x1 + o; ...
        q, k, v = b["qkv"][:width], b["qkv"][width:2 * width], b["qkv"][2 * width:]
        backend.copy(b["x1"], b["x"])
        backend.add_rms_norm(b["x1"].view(1, -1), b["delta"].view(1, -1), n1, b["h"].view(1, -1), 1e-6)
        backend.gemv_bf16(b["h"], wqkv, b["qkv"])
        backend.rope_qk_step(q, heads, k, heads, hd, b["state"], inv, None, 0)
        backend.append_step(b["kc"], k, b["state"])
        backend.append_step(b["vc"], v, b["state"])
        backend.attend_step(q, b["kc"], b["vc"], heads, hd, None, scale, b["state"], b["scratch"], b["attn"])
        backend.gemv_bf16(b["attn"], wo, b["o"])
        backend.copy(b["x2"], b["x1"])
        backend.add_rms_norm(b["x2"].view(1, -1), b["o"].view(1, -1), n2, b["h"].view(1, -1), 1e-6)
        backend.gemv_bf16(b["h"], wg, b["g"])
        backend.gemv_bf16(b["h"], wu, b["u"])
        backend.silu_mul(b["g"], b["u"])
        backend.gemv_bf16(b["g"], wd, b["out"])

    def fused(b):
        q, k, v = b["qkv"][:width], b["qkv"][width:2 * width], b["qkv"][2 * width:]
        backend.add_rms_norm_gemv_bf16(b["x"], wqkv, b["qkv"], delta=b["delta"], x_out=b["x1"], w_norm=n1)
        backend.attend_rope_kv_step(q, k, v, b["kc"], b["vc"], heads, hd, None, scale, b["state"], inv, None, 0,
                                    b["scratch"], b["attn"])
        backend.gemv_bf16(b["attn"], wo, b["o"])
        backend.add_rms_norm_swiglu_gemv_bf16(b["x1"], wg, wu, b["act"], delta=b["o"], x_out=b["x2"], w_norm=n2)
        backend.gemv_bf16(b["act"], wd, b["out"])

    torch.cuda.synchronize()
    graphs = []
    for b, body in ((A, unfused), (B, fused)):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            body(b)
        graphs.append(g)
    for step, pos in enumerate([0, 1, 37, 200, 511, 600]):
        xv, dv = normal(350 + step, hidden), normal(360 + step, hidden)
        for b in (A, B):
            b["x"].copy_(dev_f32(xv))
            b["delta"].copy_(dev_f32(dv))
            b["state"].copy_(torch.tensor([0, pos, pos, 0, -1]))
        torch.cuda.synchronize()
        for g in graphs:
            g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(A["out"]), bits(B["out"])), f"layer output at pos {pos}"
        assert np.array_equal(bits(A["x2"]), bits(B["x2"])), f"residual at pos {pos}"
        assert np.array_equal(bits(A["kc"]), bits(B["kc"])) and np.array_equal(bits(A["vc"]), bits(B["vc"]))
        assert np.array_equal(bits(A["g"]), bits(B["act"]))


@pytest.mark.parametrize("dtype,cols,with_delta", [("bf16", 2048, True), ("bf16", 2048, False), ("f32", 1280, True),
                                                   ("f32", 1280, False), ("bf16", 1283, True), ("f32", 8192, True)])
def test_embed_add_rms_norm_matches_unfused(backend, dtype, cols, with_delta):
    vocab = 3000
    table = weights_bf16(370, (vocab, cols), 0.02)
    w = dev_f32(1 + 0.02 * normal(371, cols))
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    delta = dev_f32(normal(372, cols)).to(tdt) if with_delta else None
    for token in (17, vocab - 1, vocab + 5):  # the last row, and one past the table: a zero row
        state = dev_i64([token, 3, 3, 0, -1])
        xu, hu = torch.empty(cols, dtype=tdt, device="cuda"), torch.empty(cols, dtype=tdt, device="cuda")
        backend.embed_step(table, state, xu)  # bounded by the table: out-of-range gives zeros
        if with_delta:
            backend.add_rms_norm(xu.view(1, -1), delta.view(1, -1), w, hu.view(1, -1), 1e-6)
        else:
            hu.copy_(xu)
            backend.rms_norm(hu.view(1, -1), w, 1e-6)
        x, h = torch.empty_like(xu), torch.empty_like(hu)
        backend.embed_add_rms_norm_step(table, state, w, x, h, delta=delta)
        view = torch.int16 if dtype == "bf16" else torch.int32
        assert torch.equal(x.view(view), xu.view(view)) and torch.equal(h.view(view), hu.view(view)), token


def test_embed_add_rms_norm_full_vocabulary_against_oracle(backend):
    """The bf16 embed + add + RMSNorm step on the model's whole table
    [128000, 2048] (500 MB, generated on the device), rows at both ends and
    the middle, against the oracle's chain (embedding row, add, RMSNorm in
    fp32): x = bf16(row + delta) exactly, h within 2 bf16 ulp; a token past
    the table reads a zero row."""
    vocab, cols = 128000, 2048
    g = torch.Generator(device="cuda").manual_seed(373)
    table = (0.02 * torch.randn(vocab, cols, device="cuda", generator=g)).to(torch.bfloat16)
    w_host = (1 + 0.02 * normal(374, cols)).astype(np.float32)
    d_bits = oracle.f32_to_bf16(normal(375, cols))
    w, delta = dev_f32(w_host), dev_bf16(d_bits)
    x, h = torch.empty(cols, dtype=torch.bfloat16, device="cuda"), torch.empty(cols, dtype=torch.bfloat16, device="cuda")
    for token in (127999, 127998, 64000, 0, 128000):
        backend.embed_add_rms_norm_step(table, dev_i64([token, 5, 5, 0, -1]), w, x, h, delta=delta)
        torch.cuda.synchronize()
        if token < vocab:
            row = oracle.bf16_to_f32(table[token].view(torch.int16).cpu().numpy().view(np.uint16))
        else:
            row = np.zeros(cols, np.float32)
        want_x, want_h = oracle.add_rms_norm(row[None], oracle.bf16_to_f32(d_bits)[None], w_host, 1e-6)
        got_x = x.view(torch.int16).cpu().numpy().view(np.uint16)
        got_h = h.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got_x, oracle.f32_to_bf16(want_x[0])), f"x at token {token}"
        assert_bf16_close(got_h, want_h[0], f"h at token {token}")
    del table


@pytest.mark.parametrize("heads,hd,cap,pos,masked", [(10, 128, 8192, 5000, False), (10, 128, 2048, 1500, True),
                                                     (2, 66, 100, 57, False), (4, 256, 10000, 9999, False)])
def test_attend_rope_kv_bf16_cache_matches_unfused(backend, heads, hd, cap, pos, masked):
    width = heads * hd
    q, k_row, v_row = dev_f32(normal(380, width)), dev_f32(normal(381, width)), dev_f32(normal(382, width))
    kc0, vc0 = oracle.f32_to_bf16(normal(383, (cap, width))), oracle.f32_to_bf16(normal(384, (cap, width)))
    inv = dev_f32(oracle.rope_inv(hd // 2, 1e4))
    mask = None
    if masked:
        m = np.where(np.random.default_rng(385).random(cap) < 0.4, -np.inf, 0).astype(np.float32)
        m[pos] = 0.0
        mask = dev_f32(m)
    state = state_of(pos)
    scale = float(1 / np.sqrt(hd))
    scratch = torch.empty(backend.attend_scratch_floats(heads, hd, cap), device="cuda")
    qq, kk = q.clone(), k_row.clone()
    kc1, vc1 = dev_bf16(kc0), dev_bf16(vc0)
    out1 = torch.empty(width, device="cuda")
    backend.rope_qk_step(qq, heads, kk, heads, hd, state, inv, None, 0)
    backend.append_step(kc1, kk, state)
    backend.append_step(vc1, v_row, state)
    backend.attend_step(qq, kc1, vc1, heads, hd, mask, scale, state, scratch, out1)
    kc2, vc2 = dev_bf16(kc0), dev_bf16(vc0)
    out2 = torch.empty(width, device="cuda")
    backend.attend_rope_kv_step(q, k_row, v_row, kc2, vc2, heads, hd, mask, scale, state, inv, None, 0, scratch, out2)
    assert np.array_equal(bits(out2), bits(out1))
    assert torch.equal(kc2.view(torch.int16), kc1.view(torch.int16))
    assert torch.equal(vc2.view(torch.int16), vc1.view(torch.int16))
    keys = pos + 1
    kf = oracle.bf16_to_f32(kc2.view(torch.int16).cpu().numpy().view(np.uint16))[:keys]
    vf = oracle.bf16_to_f32(vc2.view(torch.int16).cpu().numpy().view(np.uint16))[:keys]
    rq = oracle.rope(host_f32(q), heads, hd, inv_tok=host_f32(inv), one_tok=pos)
    want = oracle.attention_one(rq, kf, vf, heads, hd, None if mask is None else host_f32(mask)[:keys], scale)
    assert_f32_close(host_f32(out2), want, 1e-5, "attend_rope_kv bf16 cache")


@pytest.mark.parametrize("heads,hd,cap,pos,bs,local,nsel,max_live,dtype", [
    (10, 128, 8192, 5000, 32, 4, 8, 384, "f32"),    # the decoder's router: 8 blocks and the window
    (10, 128, 8192, 5000, 32, 4, 8, 384, "bf16"),
    (10, 128, 4096, 4095, 64, 1, 32, 2112, "f32"),  # 33 segments, the step at the cache's end
    (10, 128, 2048, 1500, 32, 0, 8, 256, "bf16"),   # no window: key pos off the segments
    (10, 128, 2048, 1500, 32, 0, 0, 32, "f32"),     # nothing live
    (10, 128, 2048, 100, 32, 4, 0, 384, "f32"),     # the window alone
    (10, 128, 2048, 1500, 32, 4, 8, 1, "f32"),      # max_live below the live keys: one split
    (2, 66, 600, 500, 16, 2, 5, 112, "f32"),        # a head that is not whole 16-byte chunks
    (4, 256, 10000, 9999, 64, 2, 12, 896, "bf16"),  # 256-wide heads past 8192 positions
    (3, 128, 512, 0, 32, 4, 0, 160, "f32")])        # the first step
def test_attend_rope_kv_segments_matches_mask(backend, heads, hd, cap, pos, bs, local, nsel, max_live, dtype):
    width = heads * hd
    g = np.random.default_rng(390 + pos)
    q, k_row, v_row = dev_f32(normal(391, width)), dev_f32(normal(392, width)), dev_f32(normal(393, width))
    inv = dev_f32(oracle.rope_inv(hd // 2, 1e4))
    remote = max(0, (pos - local * bs + 1) // bs) if local else pos // bs + 1
    blocks = np.sort(g.choice(remote, size=min(nsel, remote), replace=False)) if remote else np.zeros(0, np.int64)
    biases = (g.standard_normal(blocks.size) * 0.7).astype(np.float32)
    segs_host = key_segments(pos, bs, local, blocks, biases)
    mask_host = np.full(cap, -np.inf, np.float32)
    mask_host[:pos + 1] = mask_from_segments(segs_host, pos)
    segs = torch.from_numpy(segs_host).cuda()
    state = state_of(pos, tok=pos, page=pos // 7)
    scale = float(1 / np.sqrt(hd))
    if dtype == "bf16":
        kc0, vc0 = oracle.f32_to_bf16(normal(394, (cap, width))), oracle.f32_to_bf16(normal(395, (cap, width)))
        mk = dev_bf16
    else:
        kc0, vc0 = normal(394, (cap, width)), normal(395, (cap, width))
        mk = dev_f32
    scratch1 = torch.empty(backend.attend_scratch_floats(heads, hd, cap), device="cuda")
    kc1, vc1 = mk(kc0), mk(vc0)
    out1 = torch.empty(width, device="cuda")
    backend.attend_rope_kv_step(q, k_row, v_row, kc1, vc1, heads, hd, dev_f32(mask_host), scale, state, inv, None, 0,
                                scratch1, out1)
    scratch2 = torch.full((backend.attend_segments_scratch_floats(heads, hd, max_live),), float("nan"), device="cuda")
    kc2, vc2 = mk(kc0), mk(vc0)
    out2 = torch.full((width,), float("nan"), device="cuda")
    backend.attend_rope_kv_step_segments(q, k_row, v_row, kc2, vc2, heads, hd, segs, max_live, scale, state, inv,
                                         None, 0, scratch2, out2)
    # a second call on the same scratch (the step's key appended again: the
    # same caches) gives the same output
    out3 = torch.full((width,), float("nan"), device="cuda")
    backend.attend_rope_kv_step_segments(q, k_row, v_row, kc2, vc2, heads, hd, segs, max_live, scale, state, inv,
                                         None, 0, scratch2, out3)
    assert np.array_equal(bits(out3), bits(out2))
    if dtype == "bf16":
        assert torch.equal(kc2.view(torch.int16), kc1.view(torch.int16))
        assert torch.equal(vc2.view(torch.int16), vc1.view(torch.int16))
        kf = oracle.bf16_to_f32(kc2.view(torch.int16).cpu().numpy().view(np.uint16))[:pos + 1]
        vf = oracle.bf16_to_f32(vc2.view(torch.int16).cpu().numpy().view(np.uint16))[:pos + 1]
    else:
        assert np.array_equal(bits(kc2), bits(kc1)) and np.array_equal(bits(vc2), bits(vc1))
        kf, vf = host_f32(kc2)[:pos + 1], host_f32(vc2)[:pos + 1]
    got = host_f32(out2)
    if int(segs_host[1]) == 0:
        assert np.array_equal(got, np.zeros(width, np.float32))  # no live key: zeros, as under an all -inf mask
        assert np.array_equal(host_f32(out1), got)
        return
    assert_f32_close(got, host_f32(out1), 1e-5, "segments against the mask")
    rq = oracle.rope(host_f32(q), heads, hd, inv_tok=host_f32(inv), one_tok=pos)
    want = oracle.attention_one(rq, kf, vf, heads, hd, mask_host[:pos + 1], scale)
    assert_f32_close(got, want, 1e-5, "segments against the oracle")


def test_attend_segments_rejects_bad_arguments(backend):
    heads, hd, cap = 2, 64, 128
    q = torch.zeros(heads * hd, device="cuda")
    kc, vc = torch.zeros(cap, heads * hd, device="cuda"), torch.zeros(cap, heads * hd, device="cuda")
    segs = torch.zeros(4 * 34, dtype=torch.int32, device="cuda")
    scratch = torch.empty(backend.attend_segments_scratch_floats(heads, hd, 64 * 32), device="cuda")  # 64 splits
    out = torch.empty(heads * hd, device="cuda")
    st = state_of(3)
    inv = dev_f32(oracle.rope_inv(hd // 2, 1e4))
    with pytest.raises(ValueError, match="max_live"):  # past the capacity
        backend.attend_rope_kv_step_segments(q, q, q, kc, vc, heads, hd, segs, cap + 1, 1.0, st, inv, None, 0,
                                             scratch, out)
    with pytest.raises(ValueError, match="max_live"):
        backend.attend_rope_kv_step_segments(q, q, q, kc, vc, heads, hd, segs, 0, 1.0, st, inv, None, 0, scratch,
                                             out)
    with pytest.raises(ValueError, match="int32"):  # float32 segments
        backend.attend_rope_kv_step_segments(q, q, q, kc, vc, heads, hd, torch.zeros(4 * 34, device="cuda"), 32, 1.0,
                                             st, inv, None, 0, scratch, out)


@pytest.mark.parametrize("heads,hd,n,nsel,max_live,with_bias", [
    (10, 128, 1280, 8, 384, False),   # the decoder's o projection, 12 splits
    (10, 128, 1280, 0, 384, True),    # the window alone: splits without keys
    (16, 128, 2048, 32, 2112, False),  # 64 splits (k 2048, four chunks per lane)
    (2, 64, 300, 3, 1, True),         # one split
    (4, 64, 77, 20, 1344, False)])    # 42 splits, three value batches
def test_attend_merge_gemv_matches_unfused(backend, heads, hd, n, nsel, max_live, with_bias):
    """The o projection that merges the attention's split records in its
    prologue: bitwise the attention's own merge launch followed by gemv_bf16,
    its merged row bitwise the attention's output."""
    width = heads * hd
    cap, bs, local = 4096, 64 if max_live > 1024 else 32, 1 if max_live > 1024 else 4
    pos = cap - 1
    g = np.random.default_rng(400 + n)
    remote = (pos - local * bs + 1) // bs
    blocks = np.sort(g.choice(remote, size=min(nsel, remote), replace=False))
    segs = torch.from_numpy(key_segments(pos, bs, local, blocks, (g.standard_normal(blocks.size) * 0.5)
                                         .astype(np.float32))).cuda()
    q, k_row, v_row = dev_f32(normal(401, width)), dev_f32(normal(402, width)), dev_f32(normal(403, width))
    kc, vc = dev_f32(normal(404, (cap, width))), dev_f32(normal(405, (cap, width)))
    inv = dev_f32(oracle.rope_inv(hd // 2, 1e4))
    state = state_of(pos, tok=pos)
    scale = float(1 / np.sqrt(hd))
    scratch = torch.empty(backend.attend_segments_scratch_floats(heads, hd, max_live), device="cuda")
    w = weights_bf16(406, (n, width))
    bias = dev_f32(normal(407, n)) if with_bias else None
    # unfused: the attention's merge into attn, then the GEMV
    attn = torch.empty(width, device="cuda")
    backend.attend_rope_kv_step_segments(q, k_row, v_row, kc, vc, heads, hd, segs, max_live, scale, state, inv, None,
                                         0, scratch, attn)
    y1 = torch.empty(n, device="cuda")
    backend.gemv_bf16(attn, w, y1, bias=bias)
    # fused: records only, then the merging GEMV
    backend.attend_rope_kv_step_segments(q, k_row, v_row, kc, vc, heads, hd, segs, max_live, scale, state, inv, None,
                                         0, scratch, None)
    y2 = torch.full((n,), float("nan"), device="cuda")
    merged = torch.full((width,), float("nan"), device="cuda")
    backend.attend_merge_gemv_bf16(scratch, heads, hd, max_live, w, y2, bias=bias, x_out=merged)
    assert np.array_equal(bits(merged), bits(attn))
    assert np.array_equal(bits(y2), bits(y1))
    with pytest.raises(ValueError):
        backend.attend_merge_gemv_bf16(scratch, heads, hd, max_live, w[:, :width - 8].contiguous(), y2)
