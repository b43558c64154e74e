"""GPU parity for the fp32 products and row moves of a prefill pass
(csrc/prefill_ops.hip) through the C ABI:

  * gemm_nt / gemm_nn (the reference's cuBLAS SGEMMs, src/backend/cuda/
    ops.cu:289-309) against float64 products of the same fp32 operands, at
    1e-5 of the largest |c| (fp32 accumulation), over ragged shapes, leading
    dimensions wider than the rows, and strided batches shaped as the
    prefill attention uses them (per-head slices of q, K and V);
  * gather_rows exactly; scatter_add_rows bitwise against the same fp32
    steps in order (dst + fp32(weight * src), row by row, repeats included).
"""

import numpy as np
import pytest

from parity import assert_f32_close, dev_f32, dev_i64, host_f32, normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def device(backend):
    if not torch.cuda.is_available() or backend.device_count() == 0:
        pytest.skip("no HIP device")
    torch.cuda.set_device(0)
    yield
    torch.cuda.synchronize()


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 5, 3), (64, 64, 16), (65, 130, 33), (300, 200, 128), (37, 4096, 16)])
def test_gemm_nt_and_nn(backend, m, n, k):
    a, b_nt, b_nn = normal(500 + m, (m, k)), normal(501 + n, (n, k)), normal(502 + k, (k, n))
    c = torch.full((m, n), float("nan"), device="cuda")
    backend.gemm_nt(m, n, k, 0.37, dev_f32(a), k, 0, dev_f32(b_nt), k, 0, c, n, 0)
    assert_f32_close(host_f32(c), (0.37 * (a.astype(np.float64) @ b_nt.T.astype(np.float64))).astype(np.float32),
                     1e-5, f"gemm_nt {m}x{n}x{k}")
    backend.gemm_nn(m, n, k, dev_f32(a), k, 0, dev_f32(b_nn), n, 0, c, n, 0)
    assert_f32_close(host_f32(c), (a.astype(np.float64) @ b_nn.astype(np.float64)).astype(np.float32), 1e-5,
                     f"gemm_nn {m}x{n}x{k}")


def test_gemm_attention_shapes(backend):
    """The prefill attention's calls: per head h, S_h = scale q_h K_h^T over
    rows x keys and O_h = P_h V_h, q/K/V rows [*, heads * hd] with head h at
    column h * hd, S/P [heads, rows, keys]."""
    heads, hd, rows, keys = 4, 32, 50, 90
    width = heads * hd
    q, kc, vc = normal(510, (rows, width)), normal(511, (keys, width)), normal(512, (keys, width))
    s = torch.empty(heads, rows, keys, device="cuda")
    scale = float(1 / np.sqrt(hd))
    backend.gemm_nt(rows, keys, hd, scale, dev_f32(q), width, hd, dev_f32(kc), width, hd, s, keys, rows * keys, heads)
    p = normal(513, (heads, rows, keys))
    o = torch.full((rows, width), float("nan"), device="cuda")
    backend.gemm_nn(rows, hd, keys, dev_f32(p), keys, rows * keys, dev_f32(vc), width, hd, o, width, hd, heads)
    q64, k64, v64 = q.astype(np.float64), kc.astype(np.float64), vc.astype(np.float64)
    for h in range(heads):
        cols = slice(h * hd, (h + 1) * hd)
        assert_f32_close(host_f32(s)[h], (scale * q64[:, cols] @ k64[:, cols].T).astype(np.float32), 1e-5,
                         f"scores head {h}")
        assert_f32_close(host_f32(o)[:, cols], (p[h].astype(np.float64) @ v64[:, cols]).astype(np.float32), 1e-5,
                         f"values head {h}")


def test_gemm_rejects_bad_leading_dimension(backend):
    a = torch.zeros(4, 8, device="cuda")
    c = torch.zeros(4, 4, device="cuda")
    with pytest.raises(ValueError):
        backend.gemm_nt(4, 4, 8, 1.0, a, 4, 0, a, 8, 0, c, 4, 0)


def test_gather_and_scatter_add_rows(backend):
    rows, cols, n = 40, 77, 25
    src = normal(520, (rows, cols))
    idx = np.random.default_rng(521).integers(0, rows, n).astype(np.int64)
    idx[3] = idx[4] = 9  # a repeated index
    out = torch.empty(n, cols, device="cuda")
    backend.gather_rows(dev_f32(src), dev_i64(idx), out)
    assert np.array_equal(host_f32(out), src[idx])
    dst0 = normal(522, (rows, cols))
    w = normal(523, n)
    part = normal(524, (n, cols))
    dst = dev_f32(dst0)
    backend.scatter_add_rows(dst, dev_i64(idx), dev_f32(w), dev_f32(part))
    want = dst0.copy()
    for i in range(n):
        want[idx[i]] = want[idx[i]] + (np.float32(w[i]) * part[i]).astype(np.float32)
    assert np.array_equal(host_f32(dst).view(np.uint32), want.view(np.uint32))
