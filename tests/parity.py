"""Tolerances and host<->device helpers shared by the GPU parity tests.

Tolerances (the parity gates of these ops):
  * gather: bit-exact.
  * fp32 ops: the reference's metric max|got - want| / max|want|
    (tests/cuda_ops_test.cpp:47-54) at most 1e-5 (1e-6 for the elementwise
    activations, as the reference's own device test asks).
  * bf16 ops: that metric at most 1e-2, and every element within 2 bf16 ulp
    of the oracle's fp32 result rounded to bf16, except elements within
    2^-21 * max|want| of the oracle in absolute terms: that is the fp32
    evaluation error of the oracle itself, reached only where a result
    cancels far below the size of its inputs (a*c - b*s near zero, or
    1 + erf(x) for x < -4), so ulp counting there measures fp32 noise.
"""

import numpy as np

import oracle


def max_rel(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(float(np.max(np.abs(want))) if want.size else 0.0, 1e-9)
    return float(np.max(np.abs(got - want))) / scale if want.size else 0.0


def _ordered(bits: np.ndarray) -> np.ndarray:
    b = bits.astype(np.int64)
    mag = b & 0x7FFF
    return np.where(b & 0x8000, -mag, mag)


def bf16_ulp_report(got_bits: np.ndarray, want: np.ndarray):
    """(worst ulp distance outside the floor, count inside the floor, max_rel)."""
    got_bits = np.asarray(got_bits, np.uint16).ravel()
    want = np.asarray(want, np.float32).ravel()
    got = oracle.bf16_to_f32(got_bits).astype(np.float64)
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    floor = np.ldexp(scale, -21)
    diff = np.abs(got - want.astype(np.float64))
    outside = diff > floor
    dist = np.abs(_ordered(got_bits) - _ordered(oracle.f32_to_bf16(want)))
    worst = int(dist[outside].max()) if np.any(outside) else 0
    return worst, int(np.count_nonzero(~outside & (dist > 2))), max_rel(got, want)


def assert_bf16_close(got_bits, want, what=""):
    worst, floored, rel = bf16_ulp_report(got_bits, want)
    assert worst <= 2 and rel <= 1e-2, f"{what}: max {worst} bf16 ulp, rel {rel:.3e} ({floored} at the fp32 floor)"
    return worst, rel


def assert_f32_close(got, want, tol=1e-5, what=""):
    rel = max_rel(got, want)
    assert rel <= tol, f"{what}: rel err {rel:.3e} > {tol:.0e}"
    return rel


# ---- torch plumbing ------------------------------------------------------------------


def dev_f32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def dev_i64(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.int64)).cuda()


def dev_bf16(bits):
    """uint16 bf16 bits -> a torch.bfloat16 CUDA tensor with the same bits."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16).cuda()


def host_bits(t) -> np.ndarray:
    """A torch.bfloat16 tensor's bits as uint16."""
    import torch

    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def host_f32(t) -> np.ndarray:
    return t.cpu().numpy()


def normal(seed, shape, scale=1.0, loc=0.0) -> np.ndarray:
    g = np.random.default_rng(seed)
    return (loc + scale * g.standard_normal(shape, dtype=np.float32)).astype(np.float32)


# ---- key segments of a routed decode step ----------------------------------------------------

MAX_KEY_SEGMENTS = 33
KEY_SEGMENT_WORDS = 4 * (1 + MAX_KEY_SEGMENTS)


def key_segments(pos, block_size, local_blocks, blocks, biases) -> np.ndarray:
    """The segments layout (int32 [KEY_SEGMENT_WORDS]) for a decode query at
    pos that keeps the given remote blocks (ascending) with their biases and
    the local window: each block clipped at the window's first key (or at
    pos), then the window with bias 0."""
    segs = np.zeros(KEY_SEGMENT_WORDS, np.int32)
    wkeys = local_blocks * block_size
    wfirst = max(pos - wkeys + 1, 0)
    wlen = pos - wfirst + 1 if wkeys > 0 else 0
    stop = wfirst if wkeys > 0 else pos + 1
    live, n = 0, 0
    for b, bias in zip(blocks, biases):
        first = b * block_size
        ln = max(0, min(first + block_size, stop) - first)
        segs[4 * (1 + n):4 * (2 + n)] = [first, ln, np.float32(bias).view(np.int32), 0]
        live += ln
        n += 1
    if wlen > 0:
        segs[4 * (1 + n):4 * (2 + n)] = [wfirst, wlen, 0, 0]
        n += 1
    segs[0], segs[1] = n, live + wlen
    return segs


def mask_from_segments(segs, pos) -> np.ndarray:
    """The key mask [pos + 1] that segments describe (-inf off them), after
    checking the layout: segments in ascending key order, none past pos, the
    live count their sum."""
    segs = np.asarray(segs, np.int32)
    n, live = int(segs[0]), int(segs[1])
    assert 0 <= n <= MAX_KEY_SEGMENTS, f"segment count {n}"
    mask = np.full(pos + 1, -np.inf, np.float32)
    total, end = 0, 0
    for g in range(n):
        first, ln = int(segs[4 * (1 + g)]), int(segs[4 * (1 + g) + 1])
        assert ln >= 0, f"segment {g} length {ln}"
        if ln == 0:
            continue
        assert first >= end and first + ln <= pos + 1, f"segment {g} [{first}, {first + ln}) after {end}, pos {pos}"
        mask[first:first + ln] = segs[4 * (1 + g) + 2:4 * (1 + g) + 3].view(np.float32)[0]
        total += ln
        end = first + ln
    assert total == live, f"live {live} against {total} keys in the segments"
    return mask
