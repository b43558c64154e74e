"""GPU parity for the prefill projection `linear` (csrc/gemm.hip, bf16 matrix
cores) through the C ABI, against the oracle's linear on the bf16-rounded
input (the reference's cuda::linear, src/backend/cuda/ops.h:14-17: x rounded
to bf16, fp32 accumulation, bias added to the finished sum).

  * small and ragged shapes (m, n not multiples of the 128 x 128 tile; k not
    a multiple of the 64-wide k step) against the oracle on every element;
  * the decoder's prefill shapes (S rows of hidden 1280 through q/k/v/router
    [4096], gate/up [2 x 6848] and down [1280 <- 6848]) against the oracle on
    a sample of rows (rows are independent, so a sampled row is checked
    exactly as in a full run) and, in full, against torch's fp32 product of
    the same bf16-rounded operands;
  * k not a multiple of 8 (the vision encoder's convolutions over 12
    channels: 108 columns) loads element by element, against the oracle;
  * m == 1 goes through the GEMV, bias or none, and bad shapes are refused;
  * plain products of at least 128 bf16 rows run through hipBLASLt
    (csrc/gemm_library.hip): against the oracle as above, against the tile
    kernels (UOCR_ROCM_GEMM=tiles) on the same operands, and bitwise equal
    from call to call.

Tolerance: 1e-5 of the largest |y| (fp32 accumulation in another order)."""

import os

import numpy as np
import pytest

import oracle
from parity import assert_f32_close, dev_bf16, dev_f32, host_f32, normal

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


@pytest.mark.parametrize("m,k,n,with_bias", [(2, 8, 3, False), (37, 200, 70, True), (128, 128, 128, False),
                                             (129, 64, 257, True), (5, 1288, 31, False), (300, 1280, 520, True),
                                             (64, 6848, 96, False), (37, 108, 16, True), (200, 12, 33, False),
                                             (5, 3, 7, True)])
def test_linear_against_the_oracle(backend, m, k, n, with_bias):
    x = normal(400 + m, (m, k))
    wb = bf16(0.05 * normal(401 + n, (n, k)))
    bias = normal(402, n) if with_bias else None
    want = oracle.linear(oracle.bf16_round(x), oracle.bf16_to_f32(wb), bias)
    y = torch.full((m, n), float("nan"), device="cuda")
    backend.linear(dev_f32(x), dev_bf16(wb), y, None if bias is None else dev_f32(bias))
    assert_f32_close(host_f32(y), want, 1e-5, f"linear m={m} k={k} n={n}")


@pytest.mark.parametrize("m,k,n", [(4096, 1280, 4096), (2048, 1280, 13696), (2048, 6848, 1280)])
def test_linear_model_shapes(backend, m, k, n):
    g = torch.Generator(device="cuda").manual_seed(m + n)
    x = torch.randn(m, k, device="cuda", generator=g)
    w = (0.03 * torch.randn(n, k, device="cuda", generator=g)).to(torch.bfloat16)
    y = torch.empty(m, n, device="cuda")
    backend.linear(x, w, y)
    torch.cuda.synchronize()
    # sampled rows against the oracle, exactly as a full run would check them
    rows = np.array([0, 1, m // 2, m - 2, m - 1] + list(np.random.default_rng(403).integers(0, m, 3)))
    xs = x[torch.from_numpy(rows).cuda()].cpu().numpy()
    wh = oracle.bf16_to_f32(w.view(torch.int16).cpu().numpy().view(np.uint16))
    want = oracle.linear(oracle.bf16_round(xs), wh)
    got = y.cpu().numpy()[rows]
    assert_f32_close(got, want, 1e-5, f"linear sampled rows m={m} k={k} n={n}")
    # every element against torch's fp32 product of the same rounded operands
    ref = torch.matmul(x.to(torch.bfloat16).float(), w.float().t().contiguous())
    assert_f32_close(y.cpu().numpy(), ref.cpu().numpy(), 1e-5, f"linear full m={m} k={k} n={n}")


@pytest.mark.parametrize("m,k,n", [(37, 200, 70), (300, 1280, 520), (129, 64, 257), (1, 128, 33), (64, 6848, 96),
                                   (40, 108, 16), (1000, 640, 384), (2048, 768, 384), (513, 128, 4096)])
def test_linear_bf16_x_is_linear_on_the_rounded_rows(backend, m, k, n):
    """x already bf16 (k a multiple of 64: tiles loaded straight into LDS;
    otherwise staged): the same sums as linear on the fp32 rows."""
    x = normal(420 + m, (m, k))
    wb = bf16(0.05 * normal(421 + n, (n, k)))
    bias = normal(422, n)
    want = oracle.linear(oracle.bf16_round(x), oracle.bf16_to_f32(wb), bias)
    if k % 8 == 0:
        xb = torch.empty(m, k, dtype=torch.bfloat16, device="cuda")
        backend.round_bf16(dev_f32(x), xb)
        assert np.array_equal(xb.view(torch.int16).cpu().numpy().view(np.uint16), bf16(x))  # nearest even
    else:
        xb = dev_bf16(bf16(x))
    y = torch.full((m, n), float("nan"), device="cuda")
    backend.linear(xb, dev_bf16(wb), y, dev_f32(bias))
    assert_f32_close(host_f32(y), want, 1e-5, f"linear bf16 x m={m} k={k} n={n}")
    y2 = torch.empty(m, n, device="cuda")
    if m > 1:
        # the same tiles on fp32 rows, within 1e-6; from 128 rows the bf16
        # rows go to the library, another summation order
        backend.linear(dev_f32(x), dev_bf16(wb), y2, dev_f32(bias))
        assert_f32_close(host_f32(y2), host_f32(y), 1e-6 if m < 128 else 1e-5, "fp32 x and bf16 x agree")


def test_linear_one_row_is_the_gemv(backend):
    k, n = 1280, 300
    x = normal(410, (1, k))
    wb = bf16(0.05 * normal(411, (n, k)))
    bias = normal(412, n)
    y1, y2 = torch.empty(1, n, device="cuda"), torch.empty(n, device="cuda")
    backend.linear(dev_f32(x), dev_bf16(wb), y1, dev_f32(bias))
    backend.gemv_bf16(dev_f32(x[0]), dev_bf16(wb), y2, dev_f32(bias))
    assert np.array_equal(host_f32(y1)[0].view(np.uint32), host_f32(y2).view(np.uint32))


def test_linear_rejects_bad_shapes(backend):
    x = torch.zeros(4, 0, device="cuda")
    w = torch.zeros(3, 0, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(4, 3, device="cuda")
    with pytest.raises(ValueError):  # k = 0
        backend.linear(x, w, y)
    x = torch.zeros(4, 17, device="cuda")[:, 1:].contiguous()
    w = torch.zeros(3, 16, dtype=torch.bfloat16, device="cuda")
    backend.linear(x, w, y)  # contiguous copies are aligned
    assert torch.count_nonzero(y) == 0


@pytest.mark.parametrize("m,k,n,fp32_x", [(257, 1024, 1024, True), (257, 4096, 1024, True), (257, 1024, 3072, False),
                                          (300, 1280, 520, True), (4096, 3072, 768, True), (5, 2048, 40, False),
                                          (257, 4096, 1024, False), (512, 1024, 4096, False), (513, 2048, 256, False)])
def test_linear_split_k_against_the_oracle(backend, m, k, n, fp32_x):
    """Products of few tiles and a long k split k over a workspace (CLIP's 257
    rows): the same sums in another order, against the oracle and against the
    unsplit product; wider products or shorter k run unsplit. bf16 x of at
    most 512 rows takes the 32-row tiles (split or not)."""
    x = normal(440 + m, (m, k))
    wb = bf16(0.03 * normal(441 + n, (n, k)))
    bias = normal(442, n)
    floats = backend.linear_workspace_floats(m, k, n)
    ws = torch.full((max(floats, 1),), float("nan"), device="cuda")
    xd = dev_f32(x)
    if not fp32_x:
        xd = torch.empty(m, k, dtype=torch.bfloat16, device="cuda")
        backend.round_bf16(dev_f32(x), xd)
    y = torch.full((m, n), float("nan"), device="cuda")
    backend.linear_ws(xd, dev_bf16(wb), y, ws, dev_f32(bias))
    rows = np.unique(np.array([0, 1, m // 2, m - 1]))
    want = oracle.linear(oracle.bf16_round(x[rows]), oracle.bf16_to_f32(wb), bias)
    assert_f32_close(host_f32(y)[rows], want, 1e-5, f"split linear m={m} k={k} n={n} ({floats} floats)")
    y1 = torch.empty(m, n, device="cuda")
    backend.linear(xd, dev_bf16(wb), y1, dev_f32(bias))
    assert_f32_close(host_f32(y), host_f32(y1), 1e-5, "split and unsplit agree")
    tiles = ((m + 127) // 128) * ((n + 127) // 128)
    if k >= 2048 and tiles < 64:
        assert floats > 0, "a product of few tiles and a long k splits"
    if m > 512 and (tiles >= 64 or k < 1024):
        assert floats == 0, "a wide product or a short k runs unsplit"
    small = torch.zeros(1, device="cuda")  # a workspace too small: the product runs unsplit
    y2 = torch.empty(m, n, device="cuda")
    backend.linear_ws(xd, dev_bf16(wb), y2, small, dev_f32(bias))
    assert np.array_equal(host_f32(y2), host_f32(y1))


@pytest.mark.parametrize("m,k,n,with_bias", [(4096, 768, 768, True), (4096, 3072, 768, True), (257, 4096, 1024, True),
                                             (257, 1024, 1024, False), (33, 100, 70, True), (1, 64, 8, True)])
def test_linear_add_is_the_product_then_the_add(backend, tiles_only, m, k, n, with_bias):
    """y += bf16 x . w^T + bias (a residual stream's projection) against the
    product into a temporary then add_inplace, bit for bit, split over k (257
    rows, k >= 1024) or not, ragged k, one row (every product on the tile
    kernels, whose sums the fused epilogue shares)."""
    x = normal(460 + m, (m, k))
    wb = bf16(0.03 * normal(461 + n, (n, k)))
    bias = dev_f32(normal(462, n)) if with_bias else None
    xb = torch.empty(m, k, dtype=torch.bfloat16, device="cuda")
    backend.round_bf16(dev_f32(x), xb)
    floats = backend.linear_workspace_floats(m, k, n)
    ws = torch.full((max(floats, 1),), float("nan"), device="cuda")
    resid = dev_f32(normal(463, (m, n)))
    t = torch.empty(m, n, device="cuda")
    backend.linear_ws(xb, dev_bf16(wb), t, ws, bias)
    want = resid.clone()
    backend.add_inplace(want, t)
    got = resid.clone()
    backend.linear_add(xb, dev_bf16(wb), got, ws, bias)
    assert torch.equal(got, want), f"m={m} k={k} n={n} ({floats} workspace floats)"


@pytest.mark.parametrize("m,k,n", [(257, 1024, 4096), (4096, 768, 3072), (1000, 128, 200), (5, 64, 40),
                                   (600, 256, 4096)])
@pytest.mark.parametrize("quick", [False, True])
def test_linear_act_is_the_product_then_the_activation(backend, tiles_only, m, k, n, quick):
    """y = bf16(act(bf16 x . w^T + bias)), an MLP's first projection with
    its activation in the epilogue (CLIP's fc1 [257 x 1024 -> 4096] and
    quick_gelu, SAM's lin1 [4096 x 768 -> 3072] and gelu_erf, few-row,
    64-row and 128-row tiles, ragged m and n): bitwise the product into fp32
    then act_to_bf16. Also the rows where act_to_bf16 itself is pinned to
    the oracle (test_gpu_vision_ops)."""
    x = normal(480 + m, (m, k))
    wb = bf16(0.05 * normal(481 + n, (n, k)))
    bias = dev_f32(normal(482, n))
    xb = torch.empty(m, k, dtype=torch.bfloat16, device="cuda")
    backend.round_bf16(dev_f32(x), xb)
    t = torch.empty(m, n, device="cuda")
    backend.linear(xb, dev_bf16(wb), t, bias)
    want = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    backend.act_to_bf16(t, want, quick=quick)
    got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    backend.linear_act(xb, dev_bf16(wb), got, bias, quick=quick)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"m={m} k={k} n={n} quick={quick}"


def test_linear_act_refuses_k_off_the_tile(backend):
    xb = torch.zeros(4, 72, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(8, 72, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(4, 8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="multiple of 64"):
        backend.linear_act(xb, w, y)


@pytest.mark.parametrize("m,k,n,y_rows", [(4900, 768, 768, 4096), (300, 128, 96, 257), (5, 64, 40, 3),
                                          (2048, 256, 4096, 1500)])
def test_linear_add_rows_scatters_the_kept_rows(backend, tiles_only, m, k, n, y_rows):
    """y[y_row[r]] += product row r for y_row[r] < y_rows (window slots back
    into their grid rows, padding slots dropped): bitwise the product, the
    kept rows gathered, then add_inplace."""
    g = np.random.default_rng(470 + m)
    x = normal(471 + m, (m, k))
    wb = bf16(0.03 * normal(472 + n, (n, k)))
    bias = dev_f32(normal(473, n))
    xb = torch.empty(m, k, dtype=torch.bfloat16, device="cuda")
    backend.round_bf16(dev_f32(x), xb)
    # a permutation of the y rows onto the first y_rows products, the rest padding
    y_row = np.full(m, y_rows, np.int64)
    y_row[g.permutation(m)[:y_rows]] = np.arange(y_rows)
    resid = dev_f32(normal(474, (y_rows, n)))
    t = torch.empty(m, n, device="cuda")
    backend.linear(xb, dev_bf16(wb), t, bias)
    kept = y_row < y_rows
    src = np.empty(y_rows, np.int64)
    src[y_row[kept]] = np.nonzero(kept)[0]
    want = resid.clone()
    backend.add_inplace(want, t[torch.from_numpy(src).cuda()].contiguous())
    got = resid.clone()
    backend.linear_add_rows(xb, dev_bf16(wb), got, torch.from_numpy(y_row).cuda(), bias)
    assert torch.equal(got, want), f"m={m} k={k} n={n} y_rows={y_rows}"


@pytest.fixture
def tiles_only():
    """UOCR_ROCM_GEMM=tiles for the test's duration: every product on the
    hand-written tile kernels."""
    old = os.environ.get("UOCR_ROCM_GEMM")
    os.environ["UOCR_ROCM_GEMM"] = "tiles"
    yield
    if old is None:
        del os.environ["UOCR_ROCM_GEMM"]
    else:
        os.environ["UOCR_ROCM_GEMM"] = old


@pytest.mark.parametrize("m,k,n,with_bias", [(4096, 1280, 4096, True), (4096, 1280, 6848, False),
                                             (4096, 6848, 1280, True), (257, 1024, 3072, True), (128, 64, 8, False),
                                             (300, 1288, 520, True), (1000, 200, 72, True)])
def test_library_linear_against_the_tiles(backend, m, k, n, with_bias, request):
    """The decoder's prefill projections, CLIP's 257-row ones and small or
    ragged shapes through hipBLASLt: against the oracle on sampled rows,
    against the tile kernels on every element, and bitwise from call to
    call."""
    x = normal(450 + m, (m, k))
    wb = bf16(0.03 * normal(451 + n, (n, k)))
    bias = normal(452, n) if with_bias else None
    xb = torch.empty(m, k, dtype=torch.bfloat16, device="cuda")
    backend.round_bf16(dev_f32(x), xb)
    wd = dev_bf16(wb)
    bd = None if bias is None else dev_f32(bias)
    y = torch.full((m, n), float("nan"), device="cuda")
    backend.linear(xb, wd, y, bd)
    rows = np.unique(np.array([0, 1, m // 3, m // 2, m - 1]))
    want = oracle.linear(oracle.bf16_round(x[rows]), oracle.bf16_to_f32(wb), bias)
    assert_f32_close(host_f32(y)[rows], want, 1e-5, f"library linear m={m} k={k} n={n}")
    y_again = torch.full((m, n), float("nan"), device="cuda")
    backend.linear(xb, wd, y_again, bd)
    assert np.array_equal(host_f32(y_again).view(np.uint32), host_f32(y).view(np.uint32))
    request.getfixturevalue("tiles_only")
    y_tiles = torch.full((m, n), float("nan"), device="cuda")
    backend.linear(xb, wd, y_tiles, bd)
    assert_f32_close(host_f32(y_tiles), host_f32(y), 1e-5, "tiles and library agree")
