"""GPU parity for the block router of sparse decode attention (csrc/route.hip)
through the C ABI, against the oracle's restatement of
src/model/block_router.cpp, attention_plan.cpp and decoder.cpp:42-56 (which
tests/test_oracle.py pins bit for bit to the reference's own code):

  * block summaries and block scores within the fp32 bar (1e-5 of the
    largest value: the device reduces in another order and uses its own
    expf);
  * the selection is index work, so it is held exactly: given the scores the
    device computed, the device's key mask marks exactly the keys the
    oracle's selection and key mask mark (-inf, 0, or a block's bias), and
    each bias is within 1e-6 (the device's logf against the host's);
  * the one-launch router half of a decode step equals the separate steps
    bitwise on the same rotated router rows, and a sequence of decode steps
    keeps the router-key cache and summaries the oracle keeps;
  * the live-key segments it lists describe exactly its key mask (bitwise,
    biases included) under several router settings.

Edge cases follow the reference's rules: no block before the window (only
the window is attended), exact score ties (the lower block first), page
restrictions, a page with no block in range and a candidate list with no
remote block (both fall back to every remote block)."""

import numpy as np
import pytest

import oracle
from parity import KEY_SEGMENT_WORDS, assert_f32_close, dev_f32, dev_i64, host_f32, mask_from_segments, normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

D, BS, LOCAL = 128, 32, 4


@pytest.fixture(scope="module", autouse=True)
def device(backend):
    if not torch.cuda.is_available() or backend.device_count() == 0:
        pytest.skip("no HIP device")
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


def state_of(pos, tok=None, page=0, query_page=-1):
    return dev_i64([0, pos, pos if tok is None else tok, page, query_page])


def oracle_z(z_dev, pos, nblk):
    """The device's raw scores in the oracle's convention: clamped for the
    blocks before the window, -1e9 for the rest."""
    last_remote = pos // BS - LOCAL
    z = np.full(nblk, -1e9, np.float32)
    if last_remote >= 0:
        z[:last_remote + 1] = np.clip(z_dev[:last_remote + 1], -1e4, 1e4)
    return z


def oracle_mask(z_dev, pos, p, lo=None, hi=None, query_page=-1):
    nblk = pos // BS + 1
    z = oracle_z(z_dev, pos, nblk)
    cand = None if lo is None else oracle.page_candidates(lo, hi, query_page, nblk)
    block, bias, valid = oracle.select_blocks(z[None], None if cand is None else cand[None], p)
    return oracle.key_mask(block, bias, valid, pos, pos + 1, p)[0]


def assert_same_route(got, want, what):
    """Exactly the same masked keys and the same window; biases within 1e-6."""
    assert got.shape == want.shape, what
    assert np.array_equal(np.isneginf(got), np.isneginf(want)), f"{what}: a different set of keys is read"
    assert np.array_equal(got == 0, want == 0), f"{what}: a different window or zero bias"
    fin = np.isfinite(want)
    assert np.max(np.abs(got[fin] - want[fin]), initial=0.0) <= 1e-6, f"{what}: bias"


@pytest.mark.parametrize("keys,bs", [(1, 32), (31, 32), (32, 32), (33, 32), (700, 32), (300, 64), (129, 16)])
def test_block_summaries(backend, keys, bs):
    rk = normal(300 + keys, (keys, D), 2.0)
    cls = normal(301, D)
    want = oracle.block_summaries(rk, cls, bs)
    out = torch.empty(want.shape, device="cuda")
    backend.block_summaries(dev_f32(rk), dev_f32(cls), bs, out)
    assert_f32_close(host_f32(out), want, 1e-5, f"block_summaries keys={keys} bs={bs}")


@pytest.mark.parametrize("pos", [0, 5, 31, 32, 95, 8191])
def test_summary_and_scores_step(backend, pos):
    cap = 8192
    rk = normal(310, (cap, D), 2.0)
    cls, rq = normal(311, D), normal(312, D, 2.0)
    want_s = oracle.block_summaries(rk[:pos + 1], cls, BS)
    summ = dev_f32(np.zeros((cap // BS, D), np.float32))
    if pos // BS > 0:  # the earlier blocks as earlier steps left them
        summ[:pos // BS] = dev_f32(want_s[:pos // BS])
    st = state_of(pos)
    backend.summary_step(dev_f32(rk), D, dev_f32(cls), BS, st, summ)
    got_s = host_f32(summ)
    assert_f32_close(got_s[pos // BS], want_s[pos // BS], 1e-5, f"summary_step pos={pos}")
    assert not got_s[pos // BS + 1:].any()  # nothing past the block of pos
    z = torch.full((cap // BS,), float("nan"), device="cuda")
    backend.scores_step(dev_f32(rq), summ, D, BS, st, z)
    nb = pos // BS + 1
    zd = host_f32(z)
    want_z = (rq.astype(np.float64) @ got_s[:nb].T.astype(np.float64)) / np.sqrt(D)
    assert_f32_close(zd[:nb], want_z, 1e-5, f"scores_step pos={pos}")
    assert np.all(np.isnan(zd[nb:]))  # only the blocks up to pos are written


def route_case(backend, pos, p, lo=None, hi=None, query_page=-1, ties=False, seed=0):
    nblk = pos // BS + 1
    z = normal(seed, nblk, 3.0)
    if ties:
        z[: min(nblk, 9)] = 1.5  # exact ties at the top
    mask = torch.full((pos + 1,), float("nan"), device="cuda")
    bmin = None if lo is None else dev_i64(lo)
    bmax = None if hi is None else dev_i64(hi)
    backend.route_step(dev_f32(z), bmin, bmax, state_of(pos, query_page=query_page), p, mask)
    return host_f32(mask), oracle_mask(z, pos, p, lo, hi, query_page)


@pytest.mark.parametrize("pos", [0, 100, 127, 160, 161, 1000, 4095, 8191, 65535])
def test_route_step_matches_the_selection(backend, pos):
    p = backend.RouteParams()
    got, want = route_case(backend, pos, p, seed=320 + pos)
    assert_same_route(got, want, f"route_step pos={pos}")
    if pos < LOCAL * BS:  # no block before the window: only the window is read
        assert np.all(got == 0)


def test_route_step_ties_pages_and_fallbacks(backend):
    p = backend.RouteParams()
    pos = 2047
    nblk = pos // BS + 1
    got, want = route_case(backend, pos, p, ties=True, seed=330)
    assert_same_route(got, want, "ties")
    # prompt blocks carrying image pages: page 1 spans blocks 10..19
    lo = np.full(40, -1, np.int64)
    hi = np.full(40, -1, np.int64)
    lo[10:20], hi[10:20] = 1, 1
    lo[20:30], hi[20:30] = 2, 3
    for qp in (1, 2, 3, 7, -1):  # 7: no block holds it; -1: unrestricted
        got, want = route_case(backend, pos, p, lo, hi, qp, seed=331 + qp)
        assert_same_route(got, want, f"query_page={qp}")
    # page 1's blocks all inside the window of a query at 767 (no remote candidate): fall back
    lo2, hi2 = np.full(24, -1, np.int64), np.full(24, -1, np.int64)
    lo2[20:24], hi2[20:24] = 1, 1
    got, want = route_case(backend, 767, p, lo2, hi2, 1, seed=340)
    assert_same_route(got, want, "no remote candidate")
    assert nblk > p.top_m


def test_route_blocks_prompt_rows(backend):
    p = backend.RouteParams()
    rows, first = 6, 1500
    keys = first + rows
    nblk = (keys + BS - 1) // BS
    z = normal(350, (rows, nblk), 3.0)
    z[2, :5] = 0.25
    qp = np.array([1, -1, 1, 2, 9, 1], np.int64)
    lo, hi = np.full(nblk, -1, np.int64), np.full(nblk, -1, np.int64)
    lo[5:15], hi[5:15] = 1, 1
    lo[15:25], hi[15:25] = 2, 2
    mask = torch.full((rows, keys), float("nan"), device="cuda")
    backend.route_blocks(dev_f32(z), first, keys, dev_i64(lo), dev_i64(hi), dev_i64(qp), -1, p, mask)
    got = host_f32(mask)
    for r in range(rows):
        pos = first + r
        zr = oracle_z(z[r], pos, nblk)
        cand = oracle.page_candidates(lo, hi, int(qp[r]), nblk)
        block, bias, valid = oracle.select_blocks(zr[None], None if cand is None else cand[None], oracle.RouterParams())
        want = oracle.key_mask(block, bias, valid, pos, keys, oracle.RouterParams())[0]
        assert_same_route(got[r], want, f"route_blocks row {r}")


def rope_tables():
    return oracle.rope_inv(D // 2 - 1, 1e4), oracle.rope_inv(1, 256.0)


def test_route_decode_step_is_the_separate_steps(backend):
    """The one-launch router half of a decode step against the separate
    summary, scores and route steps on its own rotated rows (bitwise), and its
    rotated rows against the oracle's router norm and page rope."""
    cap, pos = 4096, 2900
    p = backend.RouteParams()
    inv_tok, inv_page = rope_tables()
    rq, rk = normal(360, D, 3.0), normal(361, D, 3.0)
    qn, kn, cls = normal(362, D, 0.05), normal(363, D, 0.05), normal(364, D)
    cache = normal(365, (cap, D), 1.5)
    summ0 = oracle.block_summaries(cache[:pos], cls, BS)
    summ_full = np.zeros((cap // BS, D), np.float32)
    summ_full[:summ0.shape[0]] = summ0
    lo, hi = np.full(80, -1, np.int64), np.full(80, -1, np.int64)
    lo[3:40], hi[3:40] = 0, 1
    st = state_of(pos, tok=pos, page=5, query_page=1)
    rkc, sm = dev_f32(cache), dev_f32(summ_full)
    mask = torch.full((cap,), float("nan"), device="cuda")
    z_out, rqk = torch.empty(cap // BS, device="cuda"), torch.empty(2 * D, device="cuda")
    segs = torch.full((KEY_SEGMENT_WORDS,), -7, dtype=torch.int32, device="cuda")
    backend.route_decode_step(dev_f32(rq), dev_f32(rk), dev_f32(qn), dev_f32(kn), 1e-6, dev_f32(inv_tok),
                              dev_f32(inv_page), 2, dev_f32(cls), rkc, sm, dev_i64(lo), dev_i64(hi), st, p, mask,
                              z_out=z_out, rqk_out=rqk, segments=segs)
    rot = host_f32(rqk)
    # the rotated rows against the oracle: router norm (fp64 sum) then the page rope
    tok, page = np.array([pos], np.int64), np.array([5], np.int64)
    want = []
    for row, w in ((rq, qn), (rk, kn)):
        nrm = oracle.router_norm(row[None], w, 1e-6)
        want.append(oracle.rope(nrm, 1, D, tok=tok, page=page, inv_tok=inv_tok, inv_page=inv_page, page_mod=2)[0])
    assert_f32_close(rot[:D], want[0], 1e-5, "rotated rq")
    assert_f32_close(rot[D:], want[1], 1e-5, "rotated rk")
    assert np.array_equal(host_f32(rkc)[pos], rot[D:])  # appended at pos
    # the separate steps on the same rotated rows: bitwise
    cache2 = cache.copy()
    cache2[pos] = rot[D:]
    sm2 = dev_f32(summ_full)
    st2 = state_of(pos, tok=pos, page=5, query_page=1)
    backend.summary_step(dev_f32(cache2), D, dev_f32(cls), BS, st2, sm2)
    z2 = torch.empty(cap // BS, device="cuda")
    backend.scores_step(dev_f32(rot[:D]), sm2, D, BS, st2, z2)
    mask2 = torch.full((cap,), float("nan"), device="cuda")
    backend.route_step(z2, dev_i64(lo), dev_i64(hi), st2, p, mask2)
    assert np.array_equal(host_f32(sm).view(np.uint32), host_f32(sm2).view(np.uint32))
    nrem = pos // BS - LOCAL + 1
    assert np.array_equal(host_f32(z_out)[:nrem].view(np.uint32), host_f32(z2)[:nrem].view(np.uint32))
    m1, m2 = host_f32(mask), host_f32(mask2)
    assert np.array_equal(m1[:pos + 1].view(np.uint32), m2[:pos + 1].view(np.uint32))
    assert np.all(np.isnan(m1[pos + 1:]))  # only keys 0..pos are written
    assert np.array_equal(mask_from_segments(segs.cpu().numpy(), pos).view(np.uint32), m1[:pos + 1].view(np.uint32))
    # and the mask is the oracle's selection on these scores
    assert_same_route(m1[:pos + 1], oracle_mask(host_f32(z_out), pos, oracle.RouterParams(), lo, hi, 1), "fused")


def test_route_decode_steps_in_sequence(backend):
    """Decode steps 0..N through the one-launch router with its own cache and
    summaries, checked each step against the oracle's routed mask over the
    oracle's cache of the rows the device appended."""
    cap, steps = 1024, 700
    p = backend.RouteParams()
    inv_tok, inv_page = rope_tables()
    qn, kn, cls = normal(370, D, 0.05), normal(371, D, 0.05), normal(372, D)
    rkc = torch.zeros(cap, D, device="cuda")
    sm = torch.zeros(cap // BS, D, device="cuda")
    mask = torch.empty(cap, device="cuda")
    z_out, rqk = torch.empty(cap // BS, device="cuda"), torch.empty(2 * D, device="cuda")
    segs = torch.empty(KEY_SEGMENT_WORDS, dtype=torch.int32, device="cuda")
    dqn, dkn, dcls, dt, dp = dev_f32(qn), dev_f32(kn), dev_f32(cls), dev_f32(inv_tok), dev_f32(inv_page)
    host_rk = np.zeros((cap, D), np.float32)
    g = np.random.default_rng(373)
    checked = 0
    for pos in range(steps):
        rq, rk = (g.standard_normal(D) * 3).astype(np.float32), (g.standard_normal(D) * 3).astype(np.float32)
        st = state_of(pos, tok=pos, page=pos // 300)
        backend.route_decode_step(dev_f32(rq), dev_f32(rk), dqn, dkn, 1e-6, dt, dp, 2, dcls, rkc, sm, None, None, st,
                                  p, mask, z_out=z_out, rqk_out=rqk, segments=segs)
        got_mask = host_f32(mask)[:pos + 1]
        assert np.array_equal(mask_from_segments(segs.cpu().numpy(), pos).view(np.uint32), got_mask.view(np.uint32)), \
            f"segments at step {pos}"
        rot = host_f32(rqk)
        host_rk[pos] = rot[D:]
        if pos % 37 == 0 or pos == steps - 1:
            summ, _ = oracle.route_one(rot[:D], host_rk[:pos + 1], pos, cls, oracle.RouterParams())
            got_s = host_f32(sm)[:summ.shape[0]]
            assert_f32_close(got_s, summ, 1e-5, f"summaries after step {pos}")
            nrem = max(0, pos // BS - LOCAL + 1)
            if nrem:
                want_z = (rot[:D].astype(np.float64) @ got_s[:nrem].T.astype(np.float64)) / np.sqrt(D)
                assert_f32_close(host_f32(z_out)[:nrem], want_z, 1e-5, f"scores at step {pos}")
            assert_same_route(host_f32(mask)[:pos + 1], oracle_mask(host_f32(z_out), pos, oracle.RouterParams()),
                              f"mask at step {pos}")
            checked += 1
    assert np.array_equal(host_f32(rkc)[:steps], host_rk[:steps])
    assert checked >= 19


@pytest.mark.parametrize("block_size,local_blocks,top_m,top_k,floor", [
    (32, 0, 16, 8, 1e-6), (32, 4, 16, 1, 1e-6), (64, 1, 32, 32, 1e-6), (16, 2, 8, 8, 0.0), (32, 2, 1, 1, 1e-6)])
def test_route_segments_describe_the_mask(backend, block_size, local_blocks, top_m, top_k, floor):
    """The live-key segments of decode steps 0..N under other router settings
    (no local window: key pos itself live only when selected; one selection;
    32 selections of 64-key blocks, 33 segments; a zero floor, whose unsupported
    selections carry a -inf bias), each step against the step's own mask
    bitwise and its live count within the most a step can keep."""
    cap, steps = 4096, 600 if block_size != 64 else 2400
    p = backend.RouteParams()
    p.block_size, p.local_blocks, p.top_m, p.top_k, p.floor = block_size, local_blocks, top_m, top_k, floor
    inv_tok, inv_page = rope_tables()
    qn, kn, cls = normal(380, D, 0.05), normal(381, D, 0.05), normal(382, D)
    rkc = torch.zeros(cap, D, device="cuda")
    sm = torch.zeros(cap // block_size, D, device="cuda")
    mask = torch.empty(cap, device="cuda")
    segs = torch.empty(KEY_SEGMENT_WORDS, dtype=torch.int32, device="cuda")
    dqn, dkn, dcls, dt, dp = dev_f32(qn), dev_f32(kn), dev_f32(cls), dev_f32(inv_tok), dev_f32(inv_page)
    g = np.random.default_rng(383)
    rows = (g.standard_normal((steps, 2, D)) * 3).astype(np.float32)
    most = (max(top_k, 1) + local_blocks) * block_size
    biggest = 0
    for pos in range(steps):
        st = state_of(pos, tok=pos, page=pos // 300)
        backend.route_decode_step(dev_f32(rows[pos, 0]), dev_f32(rows[pos, 1]), dqn, dkn, 1e-6, dt, dp, 2, dcls, rkc,
                                  sm, None, None, st, p, mask, segments=segs)
        if pos % 7 and pos < steps - 40:
            continue
        hs = segs.cpu().numpy()
        got_mask = host_f32(mask)[:pos + 1]
        assert np.array_equal(mask_from_segments(hs, pos).view(np.uint32), got_mask.view(np.uint32)), \
            f"segments at step {pos}"
        assert int(hs[1]) <= most
        biggest = max(biggest, int(hs[0]))
    if block_size == 64:
        assert biggest == top_k + local_blocks  # every selection and the window listed


def test_route_rejects_bad_shapes(backend):
    p = backend.RouteParams(top_m=33)
    z, mask = torch.zeros(64, device="cuda"), torch.zeros(64, device="cuda")
    with pytest.raises(ValueError, match="top_m above 32"):
        backend.route_step(z, None, None, state_of(10), p, mask)
    with pytest.raises(ValueError, match="d must be a multiple of 4"):
        backend.block_summaries(torch.zeros(10, 6, device="cuda"), torch.zeros(6, device="cuda"), 32,
                                torch.zeros(6, device="cuda"))
    with pytest.raises(ValueError, match="block_size must be in"):
        backend.block_summaries(torch.zeros(10, 8, device="cuda"), torch.zeros(8, device="cuda"), 65,
                                torch.zeros(8, device="cuda"))
