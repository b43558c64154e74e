"""GPU parity of the mixture-of-experts decode ops (src/backend/cuda/ops.h:
77-90): the gate's top-k against the oracle's routing rule
(src/model/feed_forward.cpp:36-53), and expert_ffn_one bitwise against the
ops it fuses (per slot the SwiGLU pair GEMV on the expert's gate/up rows
and the GEMV on its down rows, summed in slot order as w * d then +) and
against the oracle's expert MLP."""

import numpy as np
import pytest

import oracle
from parity import assert_f32_close, dev_bf16, dev_f32, dev_i64, host_f32, normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def device(backend):
    if not torch.cuda.is_available() or backend.device_count() == 0:
        pytest.skip("no HIP device")
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


def topk(backend, logits, k):
    rows = logits.shape[0]
    ids = torch.empty(rows, k, dtype=torch.int64, device="cuda")
    w = torch.empty(rows, k, device="cuda")
    backend.expert_topk(dev_f32(logits), k, ids, w)
    return ids.cpu().numpy(), host_f32(w)


@pytest.mark.parametrize("rows,experts,k", [(1, 64, 6), (7, 128, 8), (300, 100, 1), (33, 8, 8), (5, 65, 3)])
def test_expert_topk_matches_oracle(backend, rows, experts, k):
    logits = normal(900 + experts, (rows, experts), 2.0)
    ids, w = topk(backend, logits, k)
    want_ids, want_w = oracle.expert_topk(logits, k)
    assert np.array_equal(ids, want_ids), f"top-{k} of {experts} over {rows} rows"
    assert_f32_close(w, want_w, 1e-6, "expert scores")


def test_expert_topk_ties_and_masked_rows(backend):
    logits = normal(910, (4, 64))
    logits[0] = 0.0  # every score ties: ids in index order
    logits[1, [5, 9, 40]] = 9.0  # a three-way tie at the top
    logits[2] = -np.inf  # a fully masked row scores every expert 0
    ids, w = topk(backend, logits, 6)
    want_ids, want_w = oracle.expert_topk(logits, 6)
    assert np.array_equal(ids, want_ids)
    assert ids[0].tolist() == [0, 1, 2, 3, 4, 5] and ids[1, :3].tolist() == [5, 9, 40]
    assert ids[2].tolist() == [0, 1, 2, 3, 4, 5] and not w[2].any()
    assert_f32_close(w, want_w, 1e-6, "expert scores")


def test_expert_topk_near_ties_against_the_host_rule(backend):
    """The prefill's experts are picked on the device with expert_topk's
    arithmetic, where the reference's prefill (rows > 1,
    cuda_decoder.cpp:158-172) picks them on the host after its CPU softmax.
    Both rank by score with the lower index on a tie, and both scores are
    monotone in the logits, so the two choices can differ only where two
    logits one or two ulp apart round to one score on one side and not on
    the other. Planted at the k-th place: exact ties agree; a pair one ulp
    apart agrees or swaps exactly that pair."""
    rows, experts, k = 256, 64, 6
    g = np.random.default_rng(920)
    logits = (g.standard_normal((rows, experts)) * 2.0).astype(np.float32)
    pairs = []
    for r in range(rows):
        order = np.argsort(-logits[r], kind="stable")
        a, b = int(order[k - 1]), int(order[k])  # the k-th and the (k+1)-th
        lo, hi = min(a, b), max(a, b)
        base = np.float32(logits[r, order[k - 1]])
        if r % 2 == 0:  # an exact tie: the lower index must win on both sides
            logits[r, lo] = logits[r, hi] = base
        else:  # one ulp apart, the higher index above
            logits[r, lo] = base
            logits[r, hi] = np.nextafter(base, np.float32(np.inf), dtype=np.float32)
        pairs.append((lo, hi))
    ids, _ = topk(backend, logits, k)
    want_ids, _ = oracle.expert_topk(logits, k)
    swaps = 0
    for r in range(rows):
        got, want = set(ids[r].tolist()), set(want_ids[r].tolist())
        if r % 2 == 0:
            assert got == want, f"row {r}: an exact tie chose differently"
        elif got != want:
            assert got ^ want == set(pairs[r]), f"row {r}: {sorted(got ^ want)} against the planted {pairs[r]}"
            swaps += 1
    assert swaps < rows // 2  # most one-ulp pairs still resolve alike


def expert_stacks(seed, experts, hidden, ffn):
    g = oracle.f32_to_bf16(normal(seed, (experts, ffn, hidden), 0.04))
    u = oracle.f32_to_bf16(normal(seed + 1, (experts, ffn, hidden), 0.04))
    d = oracle.f32_to_bf16(normal(seed + 2, (experts, hidden, ffn), 0.04))
    return g, u, d


@pytest.mark.parametrize("hidden,ffn,experts,k,bad", [(1280, 896, 64, 6, False), (64, 24, 5, 3, False),
                                                       (256, 512, 16, 8, True), (2048, 1024, 8, 8, False),
                                                       (128, 2048, 4, 4, False)])
def test_expert_ffn_one_matches_its_parts_and_the_oracle(backend, hidden, ffn, experts, k, bad):
    g, u, d = expert_stacks(920 + hidden, experts, hidden, ffn)
    dg, du, dd = dev_bf16(g), dev_bf16(u), dev_bf16(d)
    x = normal(930, hidden)
    rng = np.random.default_rng(931 + k)
    ids = rng.choice(experts, size=k, replace=False).astype(np.int64)
    if bad:
        ids[2] = experts + 3  # outside the stack: the slot contributes nothing
    wts = rng.uniform(0.01, 0.3, k).astype(np.float32)
    scratch = torch.empty(backend.expert_scratch_floats(k, ffn), device="cuda")
    out = torch.empty(hidden, device="cuda")
    backend.expert_ffn_one(dev_f32(x), dg, du, dd, dev_i64(ids), dev_f32(wts), scratch, out)
    got = host_f32(out)
    # the parts, on the device: per slot the SwiGLU pair GEMV and the down GEMV
    total = np.zeros(hidden, np.float32)
    want_parts = []
    for j in range(k):
        if not 0 <= ids[j] < experts:
            continue
        e = int(ids[j])
        act = torch.empty(ffn, device="cuda")
        backend.add_rms_norm_swiglu_gemv_bf16(dev_f32(x), dg[e], du[e], act)
        dj = torch.empty(hidden, device="cuda")
        backend.gemv_bf16(act, dd[e], dj)
        total = total + np.float32(wts[j]) * host_f32(dj)
        want_parts.append((e, j))
    assert np.array_equal(got.view(np.uint32), total.view(np.uint32)), f"expert_ffn_one {hidden}x{ffn} k={k}"
    # the oracle's expert MLP, with x and act rounded to bf16 as the device rounds them
    xb = oracle.bf16_round(x)
    want = np.zeros(hidden, np.float32)
    for e, j in want_parts:
        gg = oracle.linear(xb[None], oracle.bf16_to_f32(g[e]))[0]
        uu = oracle.linear(xb[None], oracle.bf16_to_f32(u[e]))[0]
        act = oracle.bf16_round(oracle.silu_mul(gg, uu))
        want = want + np.float32(wts[j]) * oracle.linear(act[None], oracle.bf16_to_f32(d[e]))[0]
    # the bf16 rounding of act can flip between two fp32 sums that differ
    # in their last bit (2^-8 of one element): 2e-4 relative
    assert_f32_close(got, want, 2e-4, "expert_ffn_one vs oracle")


def test_expert_ffn_one_rejects_bad_shapes(backend):
    x = torch.zeros(64, device="cuda")
    g = torch.zeros(4, 24, 64, dtype=torch.bfloat16, device="cuda")
    d = torch.zeros(4, 64, 24, dtype=torch.bfloat16, device="cuda")
    ids, w = dev_i64([0, 1]), dev_f32([0.5, 0.5])
    out = torch.empty(64, device="cuda")
    with pytest.raises(ValueError):  # scratch too small
        backend.expert_ffn_one(x, g, g, d, ids, w, torch.empty(10, device="cuda"), out)
    with pytest.raises(ValueError):  # k above 8
        backend.expert_ffn_one(x, g, g, d, dev_i64(list(range(4)) * 3), dev_f32([0.1] * 12),
                               torch.empty(12 * 24, device="cuda"), out)


def test_expert_ffn_one_adds_base_last(backend):
    """out = base + the routed sum, bitwise the shared experts' output and
    add_inplace of the routed sum (src/model/cuda/cuda_decoder.cpp:149-151),
    also with base and out the same buffer."""
    hidden, ffn, experts, k = 1280, 896, 16, 6
    g, u, d = expert_stacks(940, experts, hidden, ffn)
    dg, du, dd = dev_bf16(g), dev_bf16(u), dev_bf16(d)
    x, base = dev_f32(normal(941, hidden)), dev_f32(normal(942, hidden))
    ids, wts = dev_i64([3, 0, 15, 7, 8, 1]), dev_f32([0.3, 0.2, 0.15, 0.1, 0.05, 0.02])
    scratch = torch.empty(backend.expert_scratch_floats(k, ffn), device="cuda")
    routed, out = torch.empty(hidden, device="cuda"), torch.empty(hidden, device="cuda")
    backend.expert_ffn_one(x, dg, du, dd, ids, wts, scratch, routed)
    backend.expert_ffn_one(x, dg, du, dd, ids, wts, scratch, out, base=base)
    want = base.clone()
    backend.add_inplace(want, routed)
    assert torch.equal(out.view(torch.int32), want.view(torch.int32))
    inplace = base.clone()
    backend.expert_ffn_one(x, dg, du, dd, ids, wts, scratch, inplace, base=inplace)
    assert torch.equal(inplace.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("n,k", [(64, 1280), (13, 37), (100, 2048)])
def test_gemv_f32_matches_oracle(backend, n, k):
    w, x, bias = normal(950, (n, k), 0.05), normal(951, k), normal(952, n)
    y = torch.empty(n, device="cuda")
    backend.gemv_f32(dev_f32(x), dev_f32(w), y)
    assert_f32_close(host_f32(y), oracle.linear(x[None], w)[0], 1e-5, f"gemv_f32 {n}x{k}")
    backend.gemv_f32(dev_f32(x), dev_f32(w), y, bias=dev_f32(bias))
    assert_f32_close(host_f32(y), oracle.linear(x[None], w, bias)[0], 1e-5, f"gemv_f32 {n}x{k} + bias")


@pytest.mark.parametrize("shared_ffn,experts", [(1792, 64), (24, 16), (512, 128)])
def test_moe_ffn_one_is_topk_shared_gemv_then_experts(backend, shared_ffn, experts):
    hidden, ffn, k = 1280, 896, 6
    if k * ffn + shared_ffn > 8192:
        ffn = 256
    g, u, d = expert_stacks(970, experts, hidden, ffn)
    dg, du, dd = dev_bf16(g), dev_bf16(u), dev_bf16(d)
    x = dev_f32(normal(971, hidden))
    act_s = dev_f32(normal(972, shared_ffn))
    sdown = dev_bf16(oracle.f32_to_bf16(normal(973, (hidden, shared_ffn), 0.04)))
    logits = dev_f32(normal(974, experts, 2.0))
    scratch = torch.empty(backend.expert_scratch_floats(k, ffn), device="cuda")
    # the parts: top k, the shared GEMV, the routed experts added to it
    ids1, w1 = torch.empty(1, k, dtype=torch.int64, device="cuda"), torch.empty(1, k, device="cuda")
    backend.expert_topk(logits.view(1, -1), k, ids1, w1)
    shared, want = torch.empty(hidden, device="cuda"), torch.empty(hidden, device="cuda")
    backend.gemv_bf16(act_s, sdown, shared)
    backend.expert_ffn_one(x, dg, du, dd, ids1.view(-1), w1.view(-1), scratch, want, base=shared)
    ids2, w2 = torch.empty(k, dtype=torch.int64, device="cuda"), torch.empty(k, device="cuda")
    got = torch.empty(hidden, device="cuda")
    backend.moe_ffn_one(x, dg, du, dd, logits, ids2, w2, act_s, sdown, scratch, got)
    assert torch.equal(ids1.view(-1), ids2) and torch.equal(w1.view(-1).view(torch.int32), w2.view(torch.int32))
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("k,ffn,experts,with_delta", [(1280, 1792, 64, True), (2048, 1408, 128, False),
                                                      (512, 20000, 5, True), (64, 24, 100, True)])
def test_swiglu_router_gemv_is_swiglu_gemv_then_gemv_f32(backend, k, ffn, experts, with_delta):
    """The shared experts' pair GEMV and the fp32 router in one launch:
    bitwise add_rms_norm_swiglu_gemv_bf16 (its act, x_out and h_out), then
    gemv_f32 on h_out (src/model/cuda/cuda_decoder.cpp:137-146)."""
    x = dev_f32(normal(980, k))
    delta = dev_f32(normal(981, k)) if with_delta else None
    w_norm = dev_f32(1 + 0.02 * normal(982, k))
    wg = dev_bf16(oracle.f32_to_bf16(normal(983, (ffn, k), 0.04)))
    wu = dev_bf16(oracle.f32_to_bf16(normal(984, (ffn, k), 0.04)))
    router = dev_f32(normal(985, (experts, k), 0.05))
    act1, x1, h1 = (torch.empty(n, device="cuda") for n in (ffn, k, k))
    backend.add_rms_norm_swiglu_gemv_bf16(x, wg, wu, act1, delta=delta, x_out=x1, w_norm=w_norm, h_out=h1)
    want = torch.empty(experts, device="cuda")
    backend.gemv_f32(h1, router, want)
    act2, x2, h2 = (torch.empty(n, device="cuda") for n in (ffn, k, k))
    got = torch.empty(experts, device="cuda")
    backend.add_rms_norm_swiglu_router_gemv_bf16(x, wg, wu, act2, router, got, delta=delta, x_out=x2, w_norm=w_norm,
                                                 h_out=h2)
    for a, b in ((act1, act2), (x1, x2), (h1, h2), (want, got)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert_f32_close(host_f32(got), oracle.linear(host_f32(h1)[None], host_f32(router))[0], 1e-5, "router logits")
    if experts <= k:
        with pytest.raises(ValueError):  # logits overlapping the input row
            backend.add_rms_norm_swiglu_router_gemv_bf16(x, wg, wu, act2, router, x[:experts], w_norm=w_norm)
