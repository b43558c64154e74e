"""uocr_rocm_attend_step_noalloc, the decode attention that allocates
nothing: through the C ABI it must give bitwise what uocr_rocm_attend_step
gives with a caller's scratch buffer (the same kernels on the same inputs),
on two calls in a row whose second is smaller than the first (the fixed
device array keeps the first call's records, which the second must not
read), and meet the oracle's attention at the fp32 bar. A shape whose
split records exceed the fixed array is refused before any launch."""

import numpy as np
import pytest

import oracle
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


def one_call(backend, heads, hd, cap, pos, mask, seed):
    width = heads * hd
    q = normal(seed, width)
    kc, vc = normal(seed + 1, (cap, width)), normal(seed + 2, (cap, width))
    scale = float(1.0 / np.sqrt(hd))
    state = dev_i64([0, pos, pos, 0, -1])
    dq, dk, dv = dev_f32(q), dev_f32(kc), dev_f32(vc)
    dmask = None if mask is None else dev_f32(mask)
    scratch = torch.empty(backend.attend_scratch_floats(heads, hd, cap), device="cuda")
    with_scratch = torch.full((width,), float("nan"), device="cuda")
    no_alloc = torch.full((width,), float("nan"), device="cuda")
    backend.attend_step(dq, dk, dv, heads, hd, dmask, scale, state, scratch, with_scratch)
    backend.attend_step_noalloc(dq, dk, dv, heads, hd, dmask, scale, state, no_alloc)
    torch.cuda.synchronize()
    keys = min(pos + 1, cap)
    want = oracle.attention_one(q, kc[:keys], vc[:keys], heads, hd, None if mask is None else mask[:keys], scale)
    return host_f32(with_scratch), host_f32(no_alloc), want


def test_noalloc_matches_the_scratch_entry_point_on_two_calls(backend):
    # the model's decode shape at 8192 positions with a routed mask, then a smaller call
    cap = 8192
    mask = np.zeros(cap, np.float32)
    mask[np.repeat(np.random.default_rng(40).random(cap // 64) < 0.5, 64)] = -np.inf
    mask[5000] = 0.0
    ref, got, want = one_call(backend, 10, 128, cap, 5000, mask, seed=41)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "first call differs from attend_step"
    assert_f32_close(got, want, 1e-5, "noalloc first call vs oracle")
    ref, got, want = one_call(backend, 4, 64, 300, 299, None, seed=51)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "second call differs from attend_step"
    assert_f32_close(got, want, 1e-5, "noalloc second call vs oracle")


def test_noalloc_refuses_records_past_the_fixed_array(backend):
    heads, hd, cap = 8192, 256, 64  # 8192 heads x 1 split x 258 floats > 1,048,576
    assert backend.attend_scratch_floats(heads, hd, cap) > 1 << 20
    q = torch.zeros(heads * hd, device="cuda")
    kv = torch.zeros(cap * heads * hd, device="cuda")
    out = torch.zeros(heads * hd, device="cuda")
    with pytest.raises(ValueError, match="fixed 1048576-float scratch array"):
        backend.attend_step_noalloc(q, kv, kv, heads, hd, None, 1.0, dev_i64([0, 0, 0, 0, -1]), out)
