#!/usr/bin/env python3
"""Benchmark of the rocm backend's fused layer ops on one MI355X.

Workloads (synthetic N(0,1) inputs, bf16 activations unless stated, fp32
norm weights; names and sizes follow the reference's headline op set):
  1  fp32 RMSNorm x [1024, 2048], w 1 + N(0, .02), eps 1e-6
  2  decode step at batch 1: embedding gather of one id from a
     [128000, 2048] bf16 table, residual add + RMSNorm (H 2048), RoPE on
     Q [16, 128] and K [4, 128] at a position in [0, 20000]
  3  prefill RoPE in place: Q [8192, 16, 128], K [8192, 4, 128], positions
     0..8191, theta 1e4, half-split
  4  vision block: LayerNorm [4096, 1024] (eps 1e-6) then exact-erf GELU
  5  MoE-layer prefill chain over 8192 tokens: residual add + RMSNorm
     [8192, 2048], SwiGLU [8192, 2 x 1408] -> [8192, 1408], RoPE as in 3
  6  prefill attention row ops: fp32 scores [10 x 4096, 4096] scaled with
     a causal mask and softmaxed per row in one pass (the two-op pair timed
     beside it); quick GELU [4096, 4096] bf16
  7  one decoder layer's decode step at batch 1 on Unlimited-OCR-2's dims
     (hidden 1280, 10 heads x 128, FFN 896, KV cache of 8192 positions):
     add+RMSNorm, bf16 GEMVs, RoPE, cache appends and split-K attention as
     one graph, fused into 6 launches (the 11-launch unfused layer beside
     it); the 129280 x 1280 LM-head GEMV on its own
  8  the prefill pass's projections on the matrix cores for a 4096-token
     prompt at the decoder's shapes (bf16 activations and weights, fp32
     sums): TFLOP/s and fraction of the 2.5 PFLOP/s dense bf16 peak
  9  the vision encoder on one 1024-pixel view (SAM ViT-B: 12 blocks, 8 in
     14 x 14 windows and 4 global over 64 x 64 tokens, neck and stride-2
     convolutions; CLIP-L: 24 layers over 257 tokens; projector to 1280),
     random bf16 weights: ms per view and TFLOP/s of its products, timed by
     the C++ encoder (tests/cpp/rocm_vision_test.cpp --time) in a child
     process

One step = one pass of a workload's op chain over one input set. The JSON
line's `value` is workload 5 (the largest, three fused ops timed as one
sequence): algorithmic HBM bytes per step / time per step. Every workload's
µs, GB/s and fraction of the 8 TB/s HBM peak are under "configs"; workload
2 is reported in µs per decode chain (eager launches and graph replay).
Beside each streaming kernel, `copy_us` is the library's own streaming copy
of the same bytes (half read, half written) and `of_copy` the kernel's
fraction of that rate: the practical ceiling at that transfer size, which
stays well under 8 TB/s for transfers of tens of MB.

Timing: each workload keeps several input sets whose total exceeds 640 MB,
more than twice the 256 MB Infinity Cache, and steps rotate through them, so
every step reads from HBM. After W untimed warm-up steps (which also bring
the GPU clocks up), the K timed steps are captured once into a HIP graph and
replayed; HIP events on the replay stream bracket each replay, with a device
synchronisation on both sides, and the median of 5 replays is reported (each
replay's time includes its one graph launch and the replay's fixed cost).
Each timed replay follows an untimed replay of the same graph on the same
stream with no host synchronisation between them, so that timing starts
with the GPU's memory system already at work: after the idle gap of a host
synchronisation, the first microseconds of a memory-bound chain run slower
(measured on workload 5 at 20 steps: 51.0 us per step timed from idle, 50.0
us behind a 256 MiB copy; 49.0-49.4 us either way at 100 steps).
Per-kernel and per-workload figures come from the same procedure with
max(K, 100) launches per replay, so the replay's fixed cost of about 10 us
is spread over at least 100 launches; the headline times exactly K steps.

cpu_baseline: the reference's CPU path for workload 5 (the oracle's
restatement of src/backend/reference/ops.cpp and src/model/page_rope.cpp,
with the reference's threading: norms over rows on one thread per CPU this
process may use, activations and rope serial) timed on this host, median
of at least 20 runs after 3 warm-ups; workloads 1-5 each carry the same
CPU figure for their own work under "cpu".
"""

import argparse
import json
import math
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBPS = 8000.0  # MI355X HBM3E
METRIC = "achieved HBM GB/s (% of MI355X peak) per fused op; µs per decode-step op chain"
ROTATE_BYTES = 640 * 2**20


def load_backend():
    from __graft_entry__ import _load_package

    return _load_package()


# ---- algorithmic bytes per launch ------------------------------------------------------------------

def bytes_rms_norm(rows, cols, elem):
    return 2 * rows * cols * elem + cols * 4                     # R x, W x, R w


def bytes_add_rms_norm(rows, cols, elem):
    return 4 * rows * cols * elem + cols * 4                     # R x, R delta, W x', W h, R w


def bytes_swiglu(rows, ffn, elem):
    return 3 * rows * ffn * elem                                 # R gate|up, W out


def bytes_rope(rows, heads, dim, elem, pos_bytes=8):
    return 2 * rows * heads * dim * elem + rows * pos_bytes     # R/W Q and K, R positions


def bytes_layer_norm(rows, cols, elem):
    return 2 * rows * cols * elem + 2 * cols * 4                 # R x, W y, R w, R b


def bytes_gelu(n, elem):
    return 2 * n * elem


def bytes_gather(rows, cols, elem_out, elem_table=2):
    return rows * (cols * elem_table + cols * elem_out + 8)      # R row, W row, R index


def bytes_softmax(rows, cols):
    return 2 * rows * cols * 4                                   # R/W x (fp32)


def bytes_scale_mask(batch, rows, cols):
    return 2 * batch * rows * cols * 4 + rows * cols * 4         # R/W x, R mask once


def bytes_gemv(n, k, bias=False):
    return n * k * 2 + k * 4 + n * 4 + (n * 4 if bias else 0)    # R w (bf16), R x, W y, R bias


def bytes_attend(keys, heads, hd, splits):
    width = heads * hd
    part = heads * splits * (hd + 2) * 4
    return 2 * keys * width * 4 + 2 * width * 4 + 2 * part       # R K and V rows, R q, W out, W+R records


def bytes_append(width):
    return 2 * width * 4


# ---- timing helpers ---------------------------------------------------------------------------------

# Launches per graph replay for the per-kernel and per-workload figures (the
# headline times exactly --steps). A replay carries a fixed cost of about
# 10 us beyond its kernels (measured: 20 launches of add+RMSNorm [8192, 2048]
# per replay 23.5 us each, 100 launches 22.9 us each; a spin kernel queued
# ahead of the replay, which hides the host's submission, changed neither),
# so a kernel's figure spreads it over at least this many launches.
KERNEL_STEPS = 100


class Timer:
    def __init__(self, torch, steps, warmup, replays=5, use_graphs=True):
        self.torch, self.steps, self.warmup, self.replays = torch, steps, warmup, replays
        self.kernel_steps = max(steps, KERNEL_STEPS)
        self.use_graphs = use_graphs

    def graph(self, step_fns, steps=None):
        """Median ms per step over `replays` replays of a graph holding
        `steps` steps (default: kernel_steps) that rotate through step_fns
        (one per input set). With graphs off (for counter collection), eager
        launches instead."""
        torch = self.torch
        steps = self.kernel_steps if steps is None else steps
        if not self.use_graphs:
            ms = self.eager(step_fns)
            return ms, ms, ms
        for i in range(self.warmup):
            step_fns[i % len(step_fns)]()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                step_fns[i % len(step_fns)]()
        g.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(self.replays):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            # an untimed replay right before the timed one, with no host
            # synchronisation between them: timing starts with the memory
            # system at work, not waking from the idle gap of the sync
            g.replay()
            start.record()
            g.replay()
            end.record()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(end) / steps)
        del g
        return statistics.median(times), min(times), max(times)

    def eager(self, step_fns):
        """ms per step for `steps` steps launched one by one from the host."""
        torch = self.torch
        for i in range(self.warmup):
            step_fns[i % len(step_fns)]()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(self.steps):
            step_fns[i % len(step_fns)]()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / self.steps


def n_sets(footprint_bytes):
    """Input sets needed so that one rotation touches more than ROTATE_BYTES."""
    return max(2, math.ceil(ROTATE_BYTES / max(footprint_bytes, 1)))


def report(name, nbytes, ms):
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"us": round(ms * 1e3, 3), "bytes": int(nbytes), "gbps": round(gbps, 1),
            "frac": round(gbps / PEAK_GBPS, 4)}


def footprint(tensors):
    return sum(t.numel() * t.element_size() for t in tensors)


def time_kernel(timer, make_set, launch):
    """Median ms per launch of `launch(set)` rotating over fresh input sets
    whose footprint together exceeds ROTATE_BYTES."""
    first = make_set()
    sets = [first] + [make_set() for _ in range(n_sets(footprint(first)) - 1)]
    ms = timer.graph([lambda s=s: launch(s) for s in sets])[0]
    del sets, first
    return ms


# ---- workloads ------------------------------------------------------------------------------------------

def bf16_randn(torch, shape, scale=1.0):
    return (torch.randn(shape, device="cuda", dtype=torch.float32) * scale).to(torch.bfloat16)


def weights(torch, cols):
    return 1 + 0.02 * torch.randn(cols, device="cuda", dtype=torch.float32)


def calibration(be, torch, timer):
    """A plain device-to-device copy of 256 MiB by the runtime's own copy
    kernel (the PMC calibration reads its counters), read + write bytes over
    time."""
    n = 64 * 2**20  # floats
    pairs = [(torch.empty(n, device="cuda"), torch.empty(n, device="cuda")) for _ in range(3)]
    for a, b in pairs:
        a.normal_()
    ms = timer.eager([lambda p=p: p[1].copy_(p[0]) for p in pairs])
    return {"workload": "device-to-device copy, 256 MiB (runtime memcpy)", "step": report("copy", 2 * 4 * n, ms)}


_CEILING_MS = {}


def copy_ceiling_ms(be, torch, timer, nbytes):
    """ms per launch of the library's streaming copy (uocr_rocm_copy, one
    16-byte chunk per thread, nontemporal) moving nbytes: half read, half
    written, over rotating sets like every other timing. No kernel that
    reads and writes that many bytes in one launch can beat it by much, so
    it is the practical ceiling at that transfer size."""
    if nbytes not in _CEILING_MS:
        n = max(4, nbytes // 8)  # floats per buffer
        _CEILING_MS[nbytes] = time_kernel(timer, lambda: (torch.empty(n, device="cuda").normal_(),
                                                          torch.empty(n, device="cuda")),
                                          lambda s: be.copy(s[1], s[0]))
    return _CEILING_MS[nbytes]


def add_copy_ceilings(be, torch, timer, configs):
    """Beside every streaming kernel of workloads 1 and 3-6: the copy of the
    same bytes (`copy_us`) and the kernel's fraction of its rate (`of_copy`)."""
    for c in ("1", "3", "4", "5", "6"):
        for k in configs.get(c, {}).get("kernels", {}).values():
            if k.get("bytes", 0) >= 2**20:
                ms = copy_ceiling_ms(be, torch, timer, k["bytes"])
                k["copy_us"] = round(ms * 1e3, 3)
                k["of_copy"] = round(ms * 1e3 / k["us"], 3)


def config1(be, torch, timer):
    rows, cols = 1024, 2048
    nbytes = bytes_rms_norm(rows, cols, 4)
    w = weights(torch, cols)
    ms = time_kernel(timer, lambda: torch.randn(rows, cols, device="cuda"), lambda x: be.rms_norm(x, w, 1e-6))
    r = report("rms_norm fp32", nbytes, ms)
    return {"workload": "fp32 RMSNorm [1024, 2048]", "step": r, "kernels": {"rms_norm_f32": r}}


def config2(be, torch, timer):
    vocab, hidden, qh, kh, dim = 128000, 2048, 16, 4, 128
    table = bf16_randn(torch, (vocab, hidden), 0.02)
    w = weights(torch, hidden)
    inv = torch.from_numpy(be.rope_inv(dim // 2, 1e4)).cuda()
    gen = torch.Generator().manual_seed(2)
    state = torch.tensor([int(torch.randint(0, vocab, (1,), generator=gen)), 0,
                          int(torch.randint(0, 20001, (1,), generator=gen)), 0, -1], dtype=torch.int64).cuda()
    x = torch.empty(hidden, dtype=torch.bfloat16, device="cuda")
    h = torch.empty_like(x)
    delta = bf16_randn(torch, hidden)
    q, k = bf16_randn(torch, qh * dim), bf16_randn(torch, kh * dim)
    chain_bytes = (bytes_gather(1, hidden, 2) + bytes_add_rms_norm(1, hidden, 2)
                   + bytes_rope(1, qh + kh, dim, 2, pos_bytes=8))

    def chain():  # the embedding gather fused with the residual add + RMSNorm: two launches
        be.embed_add_rms_norm_step(table, state, w, x, h, delta=delta)
        be.rope_qk_step(q, qh, k, kh, dim, state, inv, None, 0)

    def chain_unfused():
        be.embed_step(table, state, x)
        be.add_rms_norm(x, delta, w, h, 1e-6)
        be.rope_qk_step(q, qh, k, kh, dim, state, inv, None, 0)

    ms_graph, lo, hi = timer.graph([chain])
    ms_eager = timer.eager([chain])
    ms_unfused = timer.graph([chain_unfused])[0]
    ms_unfused_eager = timer.eager([chain_unfused])
    kern = {}
    kern["embed_add_rms_norm_step_bf16"] = report("gather+add+norm", bytes_gather(1, hidden, 2) + 2 * hidden * 2,
                                                  timer.graph([lambda: be.embed_add_rms_norm_step(
                                                      table, state, w, x, h, delta=delta)])[0])
    kern["embed_step_bf16"] = report("gather", bytes_gather(1, hidden, 2),
                                     timer.graph([lambda: be.embed_step(table, state, x)])[0])
    kern["add_rms_norm_bf16"] = report("add_rms_norm", bytes_add_rms_norm(1, hidden, 2),
                                       timer.graph([lambda: be.add_rms_norm(x, delta, w, h, 1e-6)])[0])
    kern["rope_qk_step_bf16"] = report("rope", bytes_rope(1, qh + kh, dim, 2, 8), timer.graph(
        [lambda: be.rope_qk_step(q, qh, k, kh, dim, state, inv, None, 0)])[0])
    return {"workload": "bf16 decode chain, batch 1: gather [128000, 2048] -> add+RMSNorm 2048 -> RoPE Q[16,128] "
                        "K[4,128] (gather fused with add+RMSNorm: 2 launches)",
            "step": report("decode chain", chain_bytes, ms_graph),
            "us_per_chain_graph": round(ms_graph * 1e3, 3), "us_per_chain_eager": round(ms_eager * 1e3, 3),
            "unfused": {"launches": 3, "us_per_chain_graph": round(ms_unfused * 1e3, 3),
                        "us_per_chain_eager": round(ms_unfused_eager * 1e3, 3)},
            "kernels": kern}


def rope_set(torch, rows, qh, kh, dim):
    return (bf16_randn(torch, (rows, qh * dim)), bf16_randn(torch, (rows, kh * dim)),
            torch.arange(rows, dtype=torch.int64, device="cuda"))


def config3(be, torch, timer):
    rows, qh, kh, dim = 8192, 16, 4, 128
    nbytes = bytes_rope(rows, qh + kh, dim, 2)
    inv = torch.from_numpy(be.rope_inv(dim // 2, 1e4)).cuda()
    ms = time_kernel(timer, lambda: rope_set(torch, rows, qh, kh, dim),
                     lambda s: be.rope_qk(s[0], qh, s[1], kh, dim, s[2], None, inv, None, 0))
    r = report("rope_qk", nbytes, ms)
    return {"workload": "bf16 prefill RoPE in place, Q [8192,16,128] K [8192,4,128]", "step": r,
            "kernels": {"rope_qk_bf16": r}}


def config4(be, torch, timer):
    rows, cols = 4096, 1024
    ln_bytes, ge_bytes = bytes_layer_norm(rows, cols, 2), bytes_gelu(rows * cols, 2)
    w, b = weights(torch, cols), 0.02 * torch.randn(cols, device="cuda")

    def step(x):
        be.layer_norm(x, w, b, 1e-6)
        be.gelu_erf(x)

    make = lambda: bf16_randn(torch, (rows, cols))  # noqa: E731
    ms = time_kernel(timer, make, step)
    ms_ln = time_kernel(timer, make, lambda x: be.layer_norm(x, w, b, 1e-6))
    ms_ge = time_kernel(timer, make, lambda x: be.gelu_erf(x))
    return {"workload": "bf16 vision LayerNorm [4096, 1024] then exact GELU",
            "step": report("ln+gelu", ln_bytes + ge_bytes, ms),
            "kernels": {"layer_norm_bf16": report("ln", ln_bytes, ms_ln),
                        "gelu_erf_bf16": report("gelu", ge_bytes, ms_ge)}}


def config5(be, torch, timer):
    rows, hidden, ffn, qh, kh, dim = 8192, 2048, 1408, 16, 4, 128
    b_norm = bytes_add_rms_norm(rows, hidden, 2)
    b_swi = bytes_swiglu(rows, ffn, 2)
    b_rope = bytes_rope(rows, qh + kh, dim, 2)
    total = b_norm + b_swi + b_rope
    w = weights(torch, hidden)
    inv = torch.from_numpy(be.rope_inv(dim // 2, 1e4)).cuda()

    def norm_set():
        return {"x": bf16_randn(torch, (rows, hidden)), "d": bf16_randn(torch, (rows, hidden)),
                "h": torch.empty(rows, hidden, dtype=torch.bfloat16, device="cuda")}

    def swiglu_set():
        return {"in": bf16_randn(torch, (rows, 2 * ffn)),
                "out": torch.empty(rows, ffn, dtype=torch.bfloat16, device="cuda")}

    def chain_set():
        s = {**norm_set(), **swiglu_set()}
        s["q"], s["k"], s["pos"] = rope_set(torch, rows, qh, kh, dim)
        return s

    def norm(s):
        be.add_rms_norm(s["x"], s["d"], w, s["h"], 1e-6)

    def swiglu(s):
        be.swiglu(s["in"], s["out"])

    def rope(s):
        be.rope_qk(s["q"], qh, s["k"], kh, dim, s["pos"], None, inv, None, 0)

    def step(s):
        norm(s)
        swiglu(s)
        rope(s)

    first = chain_set()
    sets = [first] + [chain_set() for _ in range(n_sets(footprint(first.values())) - 1)]
    # the headline: exactly --steps steps per replay
    ms, lo, hi = timer.graph([lambda s=s: step(s) for s in sets], steps=timer.steps)
    ms_eager = timer.eager([lambda s=s: step(s) for s in sets])
    nsets = len(sets)
    del sets, first
    kern = {
        "add_rms_norm_bf16": report("add_rms_norm", b_norm, time_kernel(
            timer, lambda: tuple(norm_set().values()),
            lambda s: be.add_rms_norm(s[0], s[1], w, s[2], 1e-6))),
        "swiglu_bf16": report("swiglu", b_swi, time_kernel(
            timer, lambda: tuple(swiglu_set().values()), lambda s: be.swiglu(s[0], s[1]))),
        "rope_qk_bf16": report("rope_qk", b_rope, time_kernel(
            timer, lambda: rope_set(torch, rows, qh, kh, dim),
            lambda s: be.rope_qk(s[0], qh, s[1], kh, dim, s[2], None, inv, None, 0))),
    }
    return {"workload": "bf16 MoE-layer prefill chain, 8192 tokens: add+RMSNorm [8192,2048] -> SwiGLU "
                        "[8192,2x1408]->[8192,1408] -> RoPE Q[8192,16,128] K[8192,4,128]",
            "step": report("chain", total, ms), "ms_range": [round(lo, 5), round(hi, 5)],
            "ms_per_step_eager": round(ms_eager, 5), "kernels": kern, "sets": nsets}


def config6(be, torch, timer):
    """Prefill attention row ops over 4096 tokens x 10 heads (fp32 scores
    [10 x 4096, 4096]): scale + causal mask + softmax as one pass (the step),
    the reference's two-op pair beside it; and the vision MLP's quick GELU."""
    heads, rows, keys = 10, 4096, 4096
    mask = torch.triu(torch.full((rows, keys), float("-inf"), device="cuda"), 1)
    make = lambda: torch.randn(heads * rows, keys, device="cuda")  # noqa: E731
    b_sm, b_mask = bytes_softmax(heads * rows, keys), bytes_scale_mask(heads, rows, keys)
    ms_fused = time_kernel(timer, make, lambda x: be.scale_mask_softmax_rows(x, 0.088, mask, heads, rows, keys))
    ms_mask = time_kernel(timer, make, lambda x: be.scale_add_mask(x, 0.088, mask, heads, rows, keys))
    ms_sm = time_kernel(timer, make, lambda x: be.softmax_rows(x))
    ms_pair = time_kernel(timer, make, lambda x: (be.scale_add_mask(x, 0.088, mask, heads, rows, keys),
                                                  be.softmax_rows(x)))
    qg_rows, qg_cols = 4096, 4096
    b_qg = bytes_gelu(qg_rows * qg_cols, 2)
    ms_qg = time_kernel(timer, lambda: bf16_randn(torch, (qg_rows, qg_cols)), lambda x: be.quick_gelu(x))
    # the decoder prefill's whole attention over the same causal mask, head
    # dim 128, in one pass: fp32 products (without and with the workspace:
    # the mask's live tiles, runs merged), and split-operand bf16 products
    # into bf16 (tile map, split tiles and merge included)
    hd = 128
    out32 = torch.empty(heads, rows, hd, device="cuda")
    out16 = torch.empty(heads, rows, hd, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(be.attention_masked_workspace_floats(heads, rows, keys, hd), device="cuda")
    qkv = lambda: tuple(torch.randn(heads, rows, hd, device="cuda") for _ in range(3))  # noqa: E731
    ws32 = torch.empty(be.attention_workspace_floats(heads, rows, keys, hd), device="cuda")
    ms_a32 = time_kernel(timer, qkv, lambda s: be.attention(s[0], s[1], s[2], out32, heads, rows, keys, hd, 0.088,
                                                            mask))
    ms_a32w = time_kernel(timer, qkv, lambda s: be.attention(s[0], s[1], s[2], out32, heads, rows, keys, hd, 0.088,
                                                             mask, workspace=ws32))
    ms_a16 = time_kernel(timer, qkv, lambda s: be.attention_masked(s[0], s[1], s[2], out16, heads, rows, keys, hd,
                                                                   0.088, mask, ws))
    flop = 4.0 * heads * hd * rows * (rows + 1) / 2  # the causal mask's live (query, key) pairs
    attn = lambda ms: {"us": round(ms * 1e3, 2), "tflops": round(flop / (ms * 1e-3) / 1e12, 1)}  # noqa: E731
    return {"workload": "prefill attention scores [10 x 4096, 4096] fp32: scale + causal mask + softmax in one "
                        "pass; quick GELU [4096, 4096] bf16",
            "step": report("scale_mask_softmax", b_mask, ms_fused),
            "pair_scale_add_mask_then_softmax": report("pair", b_sm + b_mask, ms_pair),
            "attention_10x4096x128_causal": {"one_pass_fp32": attn(ms_a32), "one_pass_fp32_ws": attn(ms_a32w),
                                             "split_bf16": attn(ms_a16),
                                             "live_flop": flop},
            "kernels": {"scale_mask_softmax_rows_f32": report("scale_mask_softmax", b_mask, ms_fused),
                        "scale_add_mask_f32": report("scale_add_mask", b_mask, ms_mask),
                        "softmax_rows_f32": report("softmax_rows", b_sm, ms_sm),
                        "quick_gelu_bf16": report("quick_gelu", b_qg, ms_qg)}}


def config7(be, torch, timer):
    """One decoder layer's decode step at batch 1 on Unlimited-OCR-2's dims
    (hidden 1280, 10 heads x 128, FFN 896), fp32 activations, bf16 weights,
    a KV cache of 8192 positions read in full (pos 8191). Input sets are
    whole layers (weights and cache), so a rotation reads like a multi-layer
    step. The step is the fused layer (6 launches); the same layer from the
    unfused ops (11 launches, the reference's op sequence) is timed beside it."""
    hidden, heads, hd, ffn, cap = 1280, 10, 128, 896, 8192
    width = heads * hd
    pos = cap - 1
    inv = torch.from_numpy(be.rope_inv(hd // 2, 1e4)).cuda()
    state = torch.tensor([0, pos, pos, 0, -1], dtype=torch.int64).cuda()
    splits_floats = be.attend_scratch_floats(heads, hd, cap)
    splits = splits_floats // (heads * (hd + 2))
    scratch = torch.empty(splits_floats, device="cuda")
    x, delta = torch.randn(hidden, device="cuda"), torch.randn(hidden, device="cuda")
    x1, x2 = torch.empty(hidden, device="cuda"), torch.empty(hidden, device="cuda")
    h = torch.empty(hidden, device="cuda")
    qkv = torch.empty(3 * width, device="cuda")
    attn, o = torch.empty(width, device="cuda"), torch.empty(hidden, device="cuda")
    gu, act = torch.empty(1, 2 * ffn, device="cuda"), torch.empty(1, ffn, device="cuda")
    w_norm = weights(torch, hidden)
    scale = 1.0 / math.sqrt(hd)
    q, k, v = qkv[:width], qkv[width:2 * width], qkv[2 * width:]

    def layer():
        return {"qkv": bf16_randn(torch, (3 * width, hidden), 0.03), "o": bf16_randn(torch, (hidden, width), 0.03),
                "gu": bf16_randn(torch, (2 * ffn, hidden), 0.03), "down": bf16_randn(torch, (hidden, ffn), 0.03),
                "kc": torch.randn(cap, width, device="cuda"), "vc": torch.randn(cap, width, device="cuda")}

    def unfused(L):
        be.add_rms_norm(x, delta, w_norm, h, 1e-6)
        be.gemv_bf16(h, L["qkv"], qkv)
        be.rope_qk_step(q, heads, k, heads, hd, state, inv, None, 0)
        be.append_step(L["kc"], k, state)
        be.append_step(L["vc"], v, state)
        be.attend_step(q, L["kc"], L["vc"], heads, hd, None, scale, state, scratch, attn)
        be.gemv_bf16(attn, L["o"], o)
        be.add_rms_norm(x, o, w_norm, h, 1e-6)
        be.gemv_bf16(h, L["gu"], gu.view(-1))
        be.swiglu(gu, act)
        be.gemv_bf16(act.view(-1), L["down"], delta)

    def fused(L):
        be.add_rms_norm_gemv_bf16(x, L["qkv"], qkv, delta=delta, x_out=x1, w_norm=w_norm)
        be.attend_rope_kv_step(q, k, v, L["kc"], L["vc"], heads, hd, None, scale, state, inv, None, 0, scratch,
                               attn)
        be.gemv_bf16(attn, L["o"], o)
        be.add_rms_norm_swiglu_gemv_bf16(x1, L["gu"][:ffn], L["gu"][ffn:], act.view(-1), delta=o, x_out=x2,
                                         w_norm=w_norm)
        be.gemv_bf16(act.view(-1), L["down"], delta)

    b = {"add_rms_norm": 2 * bytes_add_rms_norm(1, hidden, 4), "gemv": (bytes_gemv(3 * width, hidden)
         + bytes_gemv(hidden, width) + bytes_gemv(2 * ffn, hidden) + bytes_gemv(hidden, ffn)),
         "rope": bytes_rope(1, 2 * heads, hd, 4), "append": 2 * bytes_append(width),
         "attend": bytes_attend(cap, heads, hd, splits), "swiglu": bytes_swiglu(1, ffn, 4)}
    total = sum(b.values())
    first = layer()
    sets = [first] + [layer() for _ in range(n_sets(footprint(first.values())) - 1)]
    ms, lo, hi = timer.graph([lambda s=s: fused(s) for s in sets])
    ms_eager = timer.eager([lambda s=s: fused(s) for s in sets])
    ms_unfused = timer.graph([lambda s=s: unfused(s) for s in sets])[0]
    ms_unfused_eager = timer.eager([lambda s=s: unfused(s) for s in sets])
    kern = {
        "attend_step_f32": report("attend", b["attend"], timer.graph(
            [lambda s=s: be.attend_step(q, s["kc"], s["vc"], heads, hd, None, scale, state, scratch, attn)
             for s in sets])[0]),
        "attend_rope_kv_step_f32": report("attend+rope+append", b["attend"] + b["append"], timer.graph(
            [lambda s=s: be.attend_rope_kv_step(q, k, v, s["kc"], s["vc"], heads, hd, None, scale, state, inv, None,
                                                0, scratch, attn) for s in sets])[0]),
        # a bf16 cache halves the key/value bytes and, at this shape, the splits (64 against 128)
        "attend_rope_kv_step_bf16_cache": report("attend+rope+append, bf16 cache", (b["attend"] + b["append"]) // 2,
                                                 time_kernel(timer, lambda: (bf16_randn(torch, (cap, width)),
                                                                             bf16_randn(torch, (cap, width))),
                                                             lambda c: be.attend_rope_kv_step(
                                                                 q, k, v, c[0], c[1], heads, hd, None, scale, state,
                                                                 inv, None, 0, scratch, attn))),
        "gemv_bf16_qkv": report("gemv qkv", bytes_gemv(3 * width, hidden), timer.graph(
            [lambda s=s: be.gemv_bf16(h, s["qkv"], qkv) for s in sets])[0]),
        "add_rms_norm_gemv_bf16_qkv": report("norm+gemv qkv", bytes_gemv(3 * width, hidden), timer.graph(
            [lambda s=s: be.add_rms_norm_gemv_bf16(x, s["qkv"], qkv, delta=delta, x_out=x1, w_norm=w_norm)
             for s in sets])[0]),
    }
    nsets = len(sets)
    del sets, first
    # the same fused layer over a bf16 key/value cache (half the cache bytes)
    def layer_bf16_kv():
        L = layer()
        L["kc"], L["vc"] = L["kc"].to(torch.bfloat16), L["vc"].to(torch.bfloat16)
        return L
    first = layer_bf16_kv()
    sets = [first] + [layer_bf16_kv() for _ in range(n_sets(footprint(first.values())) - 1)]
    ms_bf16_kv = timer.graph([lambda s=s: fused(s) for s in sets])[0]
    total_bf16_kv = total - (b["attend"] + b["append"]) // 2
    del sets, first
    lm_n, lm_k = 129280, 1280
    xl, yl = torch.randn(lm_k, device="cuda"), torch.empty(lm_n, device="cuda")
    kern["gemv_bf16_lm_head"] = report("gemv lm head", bytes_gemv(lm_n, lm_k), time_kernel(
        timer, lambda: bf16_randn(torch, (lm_n, lm_k), 0.03), lambda w: be.gemv_bf16(xl, w, yl)))
    kern["expert_ffn_one_6_of_64"] = expert_ffn(be, torch, timer, hidden, ffn, 64, 6)
    whole = decode_step_12(be, torch, timer, hidden, heads, hd, ffn, cap, scratch, b, lm_n)
    return {"workload": "fp32 decode layer at batch 1, hidden 1280, 10 heads x 128, FFN 896, KV cache 8192, fused "
                        "(6 launches): add+RMSNorm+GEMV qkv -> RoPE+append+attend (2) -> GEMV o -> add+RMSNorm+GEMV "
                        "gate|up+SwiGLU -> GEMV down",
            "step": report("decode layer", total, ms), "us_per_layer_graph": round(ms * 1e3, 3),
            "us_per_layer_eager": round(ms_eager * 1e3, 3), "ms_range": [round(lo, 5), round(hi, 5)],
            "unfused": {"launches": 11, "us_per_layer_graph": round(ms_unfused * 1e3, 3),
                        "us_per_layer_eager": round(ms_unfused_eager * 1e3, 3)},
            "bf16_kv_cache": {"step": report("decode layer, bf16 cache", total_bf16_kv, ms_bf16_kv),
                              "us_per_layer_graph": round(ms_bf16_kv * 1e3, 3)},
            "bytes_by_op": b, "attend_splits": splits, "kernels": kern, "sets": nsets,
            "decode_step_12_layers": whole}


PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak


def config8(be, torch, timer):
    """The prefill pass's projections on the matrix cores (`linear` over bf16
    activations, fp32 sums and output) at Unlimited-OCR-2's decoder shapes for
    a 4096-token prompt: q/k/v + router q/k [4096 <- 1280], o [1280 <- 1280],
    the dense FFN's gate and up stacked [2 x 6848 <- 1280] (one product, as
    the prompt pass forms them) and down [1280 <- 6848], the shared experts'
    gate/up [2 x 1792 <- 1280] and down [1280 <- 1792]; gate and up apart
    [6848 <- 1280] are timed beside them. Each GEMM is timed on its own over
    fresh weight sets; the step is one dense layer's projections in
    sequence: qkv+router, o, gate+up, down."""
    rows, hidden = 4096, 1280
    shapes = {"qkv_router": (4096, 1280), "o": (1280, 1280), "gate_up": (2 * 6848, 1280), "down": (1280, 6848),
              "gate": (6848, 1280), "up": (6848, 1280), "shared_gate_up": (2 * 1792, 1280),
              "shared_down": (1280, 1792)}
    xs = {k: bf16_randn(torch, (rows, k)) for k in {1280, 6848, 1792}}
    ys = {n: torch.empty(rows, n, device="cuda") for n in {4096, 1280, 6848, 2 * 6848, 2 * 1792}}
    kern = {}
    total_flop, total_us = 0.0, 0.0
    for name, (n, k) in shapes.items():
        ms = time_kernel(timer, lambda n=n, k=k: (bf16_randn(torch, (n, k), 0.03),),
                         lambda w, n=n, k=k: be.linear(xs[k], w[0], ys[n]))
        flop = 2.0 * rows * n * k
        tf = flop / (ms * 1e-3) / 1e12
        kern[name] = {"us": round(ms * 1e3, 2), "tflops": round(tf, 1), "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                      "m": rows, "n": n, "k": k}
        if name in ("qkv_router", "o", "gate_up", "down"):
            total_flop += flop
            total_us += ms * 1e3
    tf = total_flop / (total_us * 1e-6) / 1e12
    return {"workload": "prefill projections of a dense decoder layer for a 4096-token prompt (bf16 activations, "
                        "bf16 weights, fp32 sums): qkv+router, o, gate+up stacked, down",
            "step": {"us": round(total_us, 2), "tflops": round(tf, 1), "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                     "bound": "mfma"},
            "kernels": kern}


def config9(be, torch, timer):
    """The vision encoder (src/model/rocm/vision.cpp) on one 1024-pixel view
    at the model's dims with random weights: the C++ encoder times 5 calls
    of encode_view (device image in, device features out) after 2 untimed
    ones, in a child process (it holds its own 0.8 GB of weights)."""
    binary = os.path.join(os.path.dirname(be.LIB_PATH), "rocm_vision_test")
    r = subprocess.run([binary, "--time", "1024", "5"], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        raise RuntimeError(f"rocm_vision_test --time failed ({r.returncode}): {r.stderr[-2000:]}")
    fig = json.loads(r.stdout.strip().splitlines()[-1])
    return {"workload": "vision encoder, one 1024-pixel view: SAM ViT-B (12 blocks) + neck + CLIP-L (24 layers) + "
                        "projector to 1280, bf16 weights, fp32 activations",
            "step": {"us": round(fig["ms_per_view"] * 1e3, 1), "ms_per_view": fig["ms_per_view"],
                     "tflop": fig["tflop_per_view"], "tflops": fig["tflops"],
                     "frac": round(fig["tflops"] / PEAK_BF16_TFLOPS, 4), "bound": "mfma"},
            "kernels": {}}


def expert_ffn(be, torch, timer, hidden, ffn, experts, k):
    """The routed experts of one decode row (expert_ffn_one) on the model's
    MoE shape: 6 of 64 experts of FFN 896 at hidden 1280, stacks of 440 MB
    rotated past the Infinity Cache, and a fresh choice of ids per stack."""
    g = torch.Generator().manual_seed(7)

    def make():
        ids = torch.randperm(experts, generator=g)[:k].to(torch.int64).cuda()
        return (bf16_randn(torch, (experts * ffn, hidden), 0.03), bf16_randn(torch, (experts * ffn, hidden), 0.03),
                bf16_randn(torch, (experts, hidden, ffn), 0.03), ids)
    x, out = torch.randn(hidden, device="cuda"), torch.empty(hidden, device="cuda")
    wts = torch.full((k,), 1.0 / k, device="cuda")
    scratch = torch.empty(be.expert_scratch_floats(k, ffn), device="cuda")
    nbytes = 3 * k * ffn * hidden * 2 + 2 * hidden * 4 + 2 * k * ffn * 4
    ms = time_kernel(timer, make, lambda s: be.expert_ffn_one(x, s[0], s[1], s[2], s[3], wts, scratch, out))
    return report("expert_ffn_one", nbytes, ms)


def bytes_route_decode(pos, d, block_size, local_blocks, prompt_blocks, mask=True, segment_words=0):
    """The router half of a decode step (route_decode_step) at pos: R rq, rk,
    both norms and head_cls; R the block's earlier router keys, W the new
    one; W the block's summary, R the remote blocks' summaries; R the prompt
    blocks' page ranges; W the key mask over keys 0..pos (when asked for) and
    the live-key segments."""
    blk = pos // block_size
    n = pos - blk * block_size + 1
    nrem = max(blk - local_blocks + 1, 0)
    return (4 * (5 * d + (n - 1) * d + d + d + nrem * d + (pos + 1 if mask else 0) + segment_words)
            + 16 * prompt_blocks)


def decode_step_12(be, torch, timer, hidden, heads, hd, ffn, cap, scratch, b, vocab, layers=12):
    """The model's whole decode step as one graph, the C++ DecodeStep's body
    (src/model/rocm/decode_step.cpp) on Unlimited-OCR-2's decoder shape
    (weights/architecture.h): the embedding row, layer 0 with a dense FFN of
    6848, layers 1-11 mixture of experts (an fp32 router over 64 experts, 6
    routed experts of FFN 896, shared experts of FFN 1792), each layer's
    attention routed by the block router (the q, k, v and router q/k
    projections in one GEMV, router norms, PageRope at (tok, page), the
    router key's append, the block summary, the scores of the 252 remote
    blocks, top-16 1.5-entmax, the key mask and the list of its live keys in
    one launch; rope of q and k, both appends and the attention over the live
    keys alone of 8192 positions), the final norm fused into the LM-head
    GEMV. The prompt's first 4096 positions are
    128 blocks of 16 pages and the query is confined to one page. Timed over
    the reference's fp32 key/value cache and over a bf16 one. The weights
    (5.8 GB) exceed the Infinity Cache many times over."""
    width = heads * hd
    scale = 1.0 / math.sqrt(hd)
    dense_ffn, experts, top_k, expert_ffn, shared_ffn = 6848, 64, 6, 896, 1792
    d, bs, local, page_mod = hd, 32, 4, 2
    params = be.RouteParams()
    pos = cap - 1
    n_tok = hd // 2 - 1
    inv_tok = torch.from_numpy(be.rope_inv(n_tok, 1e4)).cuda()
    inv_page = torch.from_numpy(be.rope_inv(1, 256.0)).cuda()
    prompt_blocks = 128
    page_of_block = torch.arange(prompt_blocks, dtype=torch.int64) // 8
    block_min, block_max = page_of_block.cuda(), page_of_block.cuda()
    state = torch.tensor([0, pos, pos - 2048, 17, 3], dtype=torch.int64).cuda()
    table = bf16_randn(torch, (vocab, hidden), 0.5)
    lm = bf16_randn(torch, (vocab, hidden), 0.03)
    final_norm = weights(torch, hidden)

    def layer(moe):
        L = {"in": weights(torch, hidden), "post": weights(torch, hidden),
             "proj": bf16_randn(torch, (3 * width + 2 * d, hidden), 0.03), "o": bf16_randn(torch, (hidden, width), 0.03),
             "rqn": 0.1 * torch.randn(d, device="cuda"), "rkn": 0.1 * torch.randn(d, device="cuda"),
             "cls": torch.randn(d, device="cuda"), "rkeys": torch.randn(cap, d, device="cuda"),
             "summ": torch.randn(cap // bs, d, device="cuda")}
        f = shared_ffn if moe else dense_ffn
        L.update({"gate": bf16_randn(torch, (f, hidden), 0.03), "up": bf16_randn(torch, (f, hidden), 0.03),
                  "down": bf16_randn(torch, (hidden, f), 0.03), "ffn": f, "moe": moe})
        if moe:
            L.update({"router": 0.05 * torch.randn(experts, hidden, device="cuda"),
                      "gs": bf16_randn(torch, (experts * expert_ffn, hidden), 0.03),
                      "us": bf16_randn(torch, (experts * expert_ffn, hidden), 0.03),
                      "ds": bf16_randn(torch, (experts, hidden, expert_ffn), 0.03)})
        return L

    Ls = [layer(i > 0) for i in range(layers)]
    xs = [torch.empty(hidden, device="cuda"), torch.empty(hidden, device="cuda")]
    h, delta = torch.empty(hidden, device="cuda"), torch.empty(hidden, device="cuda")
    proj = torch.empty(3 * width + 2 * d, device="cuda")
    attn, o, mask = torch.empty(width, device="cuda"), torch.empty(hidden, device="cuda"), torch.empty(cap, device="cuda")
    act, logits = torch.empty(dense_ffn, device="cuda"), torch.empty(vocab, device="cuda")
    ids, wts = torch.empty(1, top_k, dtype=torch.int64, device="cuda"), torch.empty(1, top_k, device="cuda")
    rlogits = torch.empty(experts, device="cuda")
    escratch = torch.empty(be.expert_scratch_floats(top_k, expert_ffn), device="cuda")
    segs = torch.empty(be.KEY_SEGMENT_WORDS, dtype=torch.int32, device="cuda")
    max_live = (max(params.top_k, 1) + params.local_blocks) * params.block_size
    seg_splits = be.attend_segments_scratch_floats(heads, hd, max_live) // (heads * (hd + 2))
    seg_scratch = torch.empty(be.attend_segments_scratch_floats(heads, hd, max_live), device="cuda")
    q, k, v = proj[:width], proj[width:2 * width], proj[2 * width:3 * width]
    rq, rk = proj[3 * width:3 * width + d], proj[3 * width + d:]

    def route(L, with_mask=False):
        # the step lists the live keys alone (the key mask is for checking)
        be.route_decode_step(rq, rk, L["rqn"], L["rkn"], 1e-6, inv_tok, inv_page, page_mod, L["cls"], L["rkeys"],
                             L["summ"], block_min, block_max, state, params, mask if with_mask else None,
                             segments=segs)

    def step():
        cur = 0
        be.embed_step(table, state, xs[cur])
        pending = None
        for L in Ls:
            be.add_rms_norm_gemv_bf16(xs[cur], L["proj"], proj, delta=pending,
                                      x_out=None if pending is None else xs[1 - cur], w_norm=L["in"])
            if pending is not None:
                cur = 1 - cur
            route(L)
            # the splits' records stay in seg_scratch; the o projection merges them
            be.attend_rope_kv_step_segments(q, k, v, L["kc"], L["vc"], heads, hd, segs, max_live, scale, state,
                                            inv_tok, inv_page, page_mod, seg_scratch, None)
            be.attend_merge_gemv_bf16(seg_scratch, heads, hd, max_live, L["o"], o)
            a = act[:L["ffn"]]
            if L["moe"]:  # the shared experts' pair GEMV and the router in one launch
                be.add_rms_norm_swiglu_router_gemv_bf16(xs[cur], L["gate"], L["up"], a, L["router"], rlogits,
                                                        delta=o, x_out=xs[1 - cur], w_norm=L["post"], h_out=h)
            else:
                be.add_rms_norm_swiglu_gemv_bf16(xs[cur], L["gate"], L["up"], a, delta=o, x_out=xs[1 - cur],
                                                 w_norm=L["post"])
            cur = 1 - cur
            if L["moe"]:
                be.moe_ffn_one(h, L["gs"], L["us"], L["ds"], rlogits, ids.view(-1), wts.view(-1), a, L["down"],
                               escratch, delta)
            else:
                be.gemv_bf16(a, L["down"], delta)
            pending = delta
        be.add_rms_norm_gemv_bf16(xs[cur], lm, logits, delta=pending, w_norm=final_norm)

    route_bytes = bytes_route_decode(pos, d, bs, local, prompt_blocks, mask=False, segment_words=be.KEY_SEGMENT_WORDS)
    # The attention reads the K and V rows of the keys the mask keeps (the
    # local window and the selected blocks, listed as segments), the
    # segments, q, and writes its out and split records; `live` is counted
    # from the route of layer 0.
    mask.fill_(float("-inf"))
    route(Ls[0], with_mask=True)
    live = int(torch.isfinite(mask).sum().item())
    assert live == int(segs[1].item()), "the segments' live count is the mask's"
    fixed_attend = bytes_attend(0, heads, hd, seg_splits)    # q, out and the split records

    def kv_bytes(elem):
        return 2 * live * width * elem + fixed_attend + 2 * width * elem + 4 * be.KEY_SEGMENT_WORDS
    proj_bytes = bytes_gemv(3 * width + 2 * d, hidden)
    attn_fixed = b["add_rms_norm"] + b["rope"] + route_bytes + proj_bytes + bytes_gemv(hidden, width)
    dense_bytes = 3 * dense_ffn * hidden * 2
    moe_bytes = 3 * shared_ffn * hidden * 2 + experts * hidden * 4 + 3 * top_k * expert_ffn * hidden * 2
    rest = bytes_gather(1, hidden, 4) + dense_bytes + (layers - 1) * moe_bytes + bytes_gemv(vocab, hidden)
    launches = 2 + 6 + 7 * (layers - 1)
    ms_route = timer.graph([lambda L=L: route(L) for L in Ls])[0]
    out = {"workload": f"the model's decode step: embedding, layer 0 dense (FFN {dense_ffn}), layers 1-{layers - 1} "
                       f"mixture of experts ({top_k} of {experts} experts of FFN {expert_ffn}, shared FFN "
                       f"{shared_ffn}, fp32 router), block-routed attention over {cap} positions (block {bs}, local "
                       f"window {local * bs}, top-{params.top_m} entmax, {params.top_k} blocks, the query confined to "
                       f"one page of a {prompt_blocks}-block prompt), PageRope (63 token pairs, 1 page pair), final "
                       f"norm + LM head [{vocab}, {hidden}]; {launches} launches; the mask keeps {live} of "
                       f"{cap} keys, and only their K/V rows are read",
           "route_decode_step": report("route_decode_step", route_bytes, ms_route), "live_keys": live}
    for name, dtype in (("fp32_cache", torch.float32), ("bf16_cache", torch.bfloat16)):
        for L in Ls:
            L["kc"] = torch.randn(cap, width, device="cuda").to(dtype)
            L["vc"] = torch.randn(cap, width, device="cuda").to(dtype)
        total = rest + layers * (attn_fixed + kv_bytes(4 if dtype == torch.float32 else 2))
        ms = timer.graph([step])[0]
        out[name] = {"step": report(f"decode step, {name}", total, ms), "us_per_token": round(ms * 1e3, 2)}
        if name == "fp32_cache":
            # one step per replay, as DecodeStep::step replays its graph once
            # per token: the replay's own start and end no longer shared
            out[name]["us_per_token_one_replay"] = round(timer.graph([step], steps=1)[0] * 1e3, 2)
        for L in Ls:
            del L["kc"], L["vc"]
    out["step"] = out["fp32_cache"]["step"]
    out["us_per_token"] = out["fp32_cache"]["us_per_token"]
    del Ls, table, lm
    return out


# ---- the CPU baseline (the reference's CPU path, restated in the oracle) ------------------------------

def _cpu_median(fn, budget_s, max_runs=200, min_runs=20):
    """Median seconds per call of fn after 3 warm-up calls, over at least
    min_runs and at most max_runs calls (as many as budget_s allows)."""
    for _ in range(3):
        fn()
    times, t_end = [], time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_workloads(budget_s, threads):
    """Workloads 1-5 on the reference's CPU path: the oracle's C restatement
    of src/backend/reference/ops.cpp, src/model/page_rope.cpp and the
    decoder's add/copy/norm chain, called on preallocated fp32 buffers (the
    reference's only CPU dtype; bf16 inputs widened) so that no copy beyond
    the reference's own is timed. Norms run over rows on `threads` threads,
    activations, rope and the add serially, as in the reference. Returns
    {workload: figures}; rates use the same algorithmic bytes as the GPU."""
    import ctypes

    import numpy as np

    import oracle

    lib = oracle.lib()
    p = lambda a: a.ctypes.data  # noqa: E731
    g = np.random.default_rng(5)
    rnd = lambda *shape: oracle.bf16_round(g.standard_normal(shape, dtype=np.float32))  # noqa: E731
    wts = lambda n: (1 + 0.02 * g.standard_normal(n)).astype(np.float32)  # noqa: E731
    inv = oracle.rope_inv(64, 1e4)
    out = {}
    oracle.set_threads(threads)

    # 1: fp32 RMSNorm [1024, 2048] in place
    x1, w1 = g.standard_normal((1024, 2048), dtype=np.float32), wts(2048)
    t, n = _cpu_median(lambda: lib.orc_rms_norm(p(x1), p(w1), 1024, 2048, 1e-6), budget_s)
    out["1"] = {"ms": round(t * 1e3, 3), "gbps": round(bytes_rms_norm(1024, 2048, 4) / t / 1e9, 3), "runs": n}

    # 2: decode chain at batch 1 (gather of one row of a [128000, 2048] table, add + RMSNorm, rope q and k)
    table = np.empty((128000, 2048), np.uint16)  # untouched rows stay unmapped
    token, pos = 77777, 12345
    table[token] = oracle.f32_to_bf16(0.02 * g.standard_normal(2048, dtype=np.float32))
    e, d2, h2, w2 = np.empty(2048, np.float32), rnd(2048), np.empty(2048, np.float32), wts(2048)
    q2, k2 = rnd(16 * 128), rnd(4 * 128)
    nul = ctypes.c_void_p()

    reps = 200  # chains per C call: the gather, add + RMSNorm and both ropes, with no Python between them
    t, n = _cpu_median(lambda: lib.orc_decode_chain(p(table), token, p(d2), p(w2), p(e), p(h2), 2048, 1e-6, p(q2), 16,
                                                    p(k2), 4, 128, pos, p(inv), 64, reps), budget_s)
    out["2"] = {"us": round(t / reps * 1e6, 3), "runs": n,
                "note": f"mean of {reps} chains per C call (one call per run)"}
    del table

    # 3: RoPE Q [8192, 16, 128], K [8192, 4, 128] in place, positions 0..8191
    q3, k3, pos3 = rnd(8192, 16 * 128), rnd(8192, 4 * 128), np.arange(8192, dtype=np.int64)

    def rope3():
        lib.orc_rope_apply(p(q3), 8192, 16, 128, p(pos3), nul, p(inv), 64, nul, 0, 0, 0, 0)
        lib.orc_rope_apply(p(k3), 8192, 4, 128, p(pos3), nul, p(inv), 64, nul, 0, 0, 0, 0)

    t, n = _cpu_median(rope3, budget_s)
    out["3"] = {"ms": round(t * 1e3, 3), "gbps": round(bytes_rope(8192, 20, 128, 2) / t / 1e9, 3), "runs": n}

    # 4: LayerNorm [4096, 1024] then GELU, in place
    x4, w4, b4 = rnd(4096, 1024), wts(1024), (0.02 * g.standard_normal(1024)).astype(np.float32)

    def vision4():
        lib.orc_layer_norm(p(x4), p(w4), p(b4), 4096, 1024, 1e-6)
        lib.orc_gelu_erf(p(x4), 4096 * 1024)

    t, n = _cpu_median(vision4, budget_s)
    out["4"] = {"ms": round(t * 1e3, 3), "runs": n,
                "gbps": round((bytes_layer_norm(4096, 1024, 2) + bytes_gelu(4096 * 1024, 2)) / t / 1e9, 3)}

    # 5: add + RMSNorm [8192, 2048], SwiGLU [8192, 2 x 1408], rope as 3
    x5, d5, w5, h5 = rnd(8192, 2048), rnd(8192, 2048), wts(2048), np.empty((8192, 2048), np.float32)
    in5, o5 = rnd(8192, 2 * 1408), np.empty((8192, 1408), np.float32)

    def chain5():
        lib.orc_add_rms_norm(p(x5), p(d5), p(w5), p(h5), 8192, 2048, 1e-6)
        lib.orc_swiglu(p(in5), p(o5), 8192, 1408)
        rope3()

    total5 = bytes_add_rms_norm(8192, 2048, 2) + bytes_swiglu(8192, 1408, 2) + bytes_rope(8192, 20, 128, 2)
    t, n = _cpu_median(chain5, budget_s)
    oracle.set_threads(1)
    t1, n1 = _cpu_median(chain5, budget_s)
    out["5"] = {"ms": round(t * 1e3, 3), "gbps": round(total5 / t / 1e9, 3), "runs": n,
                "ms_1_thread": round(t1 * 1e3, 3), "gbps_1_thread": round(total5 / t1 / 1e9, 3)}
    return out


def host_cpu():
    """The host's CPU as this process sees it: the model string, the online
    processor count (what std::thread::hardware_concurrency reports, the
    reference's default thread count, src/backend/reference/ops.cpp:15) and
    the CPUs this process may run on."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "nproc": os.cpu_count() or 1, "affinity": len(os.sched_getaffinity(0))}


def cpu_baseline(cpu, threads, info):
    """The top-level cpu_baseline object: workload 5 from cpu_workloads."""
    c = cpu["5"]
    return {"value": c["gbps"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"workload 5 in full (8192 tokens), median of {c['runs']} chains after 3 warm-ups on "
                      f"preallocated fp32 buffers; norms on {threads} threads (the CPUs this process may use), "
                      f"activations and rope serial as in the reference",
            "cpu_model": info["model"], "nproc": info["nproc"], "affinity_cpus": info["affinity"],
            "ms_per_chain": c["ms"], "ms_per_chain_1_thread": c["ms_1_thread"], "value_1_thread": c["gbps_1_thread"]}


# ---- rocprofv3 summaries -------------------------------------------------------------------------------

PROFILES = os.path.join(ROOT, "profiles")
TRAFFIC_FILE = os.path.join(PROFILES, "pmc_traffic_workloads3_to_6.md")
COPY_KERNEL = "__amd_rocclr_copyBuffer"
COPY_BYTES = 256 * 2**20  # the calibration copy: 256 MiB read and 256 MiB written per dispatch


def _kernel_label(name):
    """A kernel's demangled name without namespaces and parameter list."""
    import re

    name = re.sub(r"uocr_rocm::\(anonymous namespace\)::", "", name).replace("void ", "").strip()
    if name.startswith("Cijk_"):  # hipBLASLt's generated kernels: keep the macro tile and the k split
        tile = re.search(r"_MT(\d+x\d+x\d+)_", name)
        gsu = re.search(r"_(GSU\d+)_", name)
        return "hipBLASLt " + " ".join(m.group(1) for m in (tile, gsu) if m)
    if name.endswith(")"):  # drop the trailing "(params)", keeping "(Norm)1"-style template arguments
        depth = 0
        for i in range(len(name) - 1, -1, -1):
            depth += {")": 1, "(": -1}.get(name[i], 0)
            if depth == 0:
                name = name[:i]
                break
    return name.strip()


def summarize_trace(trace_dir):
    """Markdown table of per-kernel durations from a --kernel-trace run."""
    import csv
    import statistics as st

    rows = list(csv.DictReader(open(os.path.join(trace_dir, "run_kernel_trace.csv"))))
    by = {}
    for r in rows:
        key = (_kernel_label(r["Kernel_Name"]), r.get("Grid_Size", r.get("Grid_Size_X", "")),
               r.get("Workgroup_Size", r.get("Workgroup_Size_X", "")))
        by.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    out = ["| kernel | grid | block | calls | mean us | median us | min us |", "|---|---|---|---|---|---|---|"]
    for (k, g, b), d in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        if k.startswith("at::") or "at::native" in k:
            continue
        out.append(f"| `{k}` | {g} | {b} | {len(d)} | {st.mean(d):.2f} | {st.median(d):.2f} | {min(d):.2f} |")
    return "\n".join(out)


# HBM-side request counters of the L2 (summed over its channels), two runs:
# the read requests by size, then all read requests and the write requests
# (at most 4 TCC counters fit one run).
PMC_PASS_READS = ("TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum")
PMC_PASS_WRITES = ("TCC_EA0_RDREQ_sum", "TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum")


def _load_counters(d):
    """{(kernel, grid): {counter: median value per dispatch}} from a --pmc run."""
    import csv
    import statistics as st

    by = {}
    for r in csv.DictReader(open(os.path.join(d, "run_counter_collection.csv"))):
        key = (_kernel_label(r["Kernel_Name"]), r.get("Grid_Size", ""))
        by.setdefault(key, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return {k: {c: st.median(v) for c, v in cs.items()} for k, cs in by.items()}


def summarize_pmc(reads_dir, writes_dir):
    """Markdown table of HBM bytes per dispatch from the L2's memory-side
    request counters, each request counted at its size: reads 32, 64 or 128
    bytes (RDREQ_32B, _64B, _128B), writes 64 bytes (WRREQ_64B) or 32 (the
    rest of WRREQ). No calibration factor: the 256 MiB copy's row checks the
    arithmetic (its read and write bytes are known), and the requests of
    unknown size (RDREQ less the three sized counts) are listed."""
    rd, wr = _load_counters(reads_dir), _load_counters(writes_dir)
    out = ["| kernel | grid | RDREQ 32B | RDREQ 64B | RDREQ 128B | unsized reads | WRREQ | WRREQ 64B | "
           "read bytes | write bytes | traffic bytes |", "|---|---|---|---|---|---|---|---|---|---|---|"]
    for key in sorted(set(rd) | set(wr)):
        k, g = key
        if k.startswith("at::") or "at::native" in k:
            continue
        r, w = rd.get(key, {}), wr.get(key, {})
        r32, r64, r128 = (r.get(c, 0.0) for c in PMC_PASS_READS)
        rall, wall, w64 = (w.get(c, 0.0) for c in PMC_PASS_WRITES)
        read_b = 32 * r32 + 64 * r64 + 128 * r128
        write_b = 64 * w64 + 32 * (wall - w64)
        unsized = rall - (r32 + r64 + r128)
        out.append(f"| `{k}` | {g} | {r32:.0f} | {r64:.0f} | {r128:.0f} | {unsized:.0f} | {wall:.0f} | {w64:.0f} | "
                   f"{read_b:.0f} | {write_b:.0f} | {read_b + write_b:.0f} |")
    return "\n".join(out)


def committed_traffic(kernel_prefix, grid):
    """HBM bytes per launch of a kernel from the committed PMC summary, or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        cells = [c.strip().strip("`") for c in line.strip().strip("|").split("|")]
        if len(cells) == 11 and cells[0].startswith(kernel_prefix) and cells[1] == str(grid):
            try:
                return int(float(cells[10]))
            except ValueError:
                return None
    return None


# ---- main ---------------------------------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--configs", default="copy,1,2,3,4,5,6,7,8,9")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly (for counter collection)")
    ap.add_argument("--summarize-trace", metavar="DIR", help="print a table from a rocprofv3 --kernel-trace run")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("READS_DIR", "WRITES_DIR"),
                    help="print a table from the two rocprofv3 --pmc runs (PMC_PASS_READS, PMC_PASS_WRITES)")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return
    if args.summarize_pmc:
        print(summarize_pmc(*args.summarize_pmc))
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: every op is row-independent and this build measures one GPU's share "
              f"(--gpus {args.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)

    import torch

    be = load_backend()
    if be.device_count() == 0 or not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    torch.manual_seed(0)
    info = be.device_info(0)
    timer = Timer(torch, args.steps, args.warmup, use_graphs=not args.no_graph)
    runners = {"1": config1, "2": config2, "3": config3, "4": config4, "5": config5, "6": config6, "7": config7,
               "8": config8, "9": config9, "copy": calibration}
    configs = {}
    for c in args.configs.split(","):
        t0 = time.time()
        configs[c] = runners[c](be, torch, timer)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        print(f"[bench] workload {c}: {json.dumps(configs[c]['step'])} ({time.time() - t0:.1f} s)", file=sys.stderr,
              flush=True)

    t0 = time.time()
    add_copy_ceilings(be, torch, timer, configs)
    torch.cuda.empty_cache()
    print(f"[bench] copy ceilings at {len(_CEILING_MS)} sizes ({time.time() - t0:.1f} s)", file=sys.stderr, flush=True)

    head = configs.get("5")
    line = {"metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "compute_dtype": "f32", "data": "synthetic N(0,1), random weights",
            "device": info["name"]}
    if head is not None:
        dom = head["kernels"]["add_rms_norm_bf16"]
        line.update({
            "value": head["step"]["gbps"], "ms_per_step": round(head["step"]["us"] / 1e3, 5),
            "config": {"workload": head["workload"], "tokens": 8192, "hidden": 2048, "ffn": 1408,
                       "q_heads": 16, "kv_heads": 4, "head_dim": 128, "bytes_per_step": head["step"]["bytes"]},
            "roofline": {"bound": "hbm", "kernel": "add_rms_norm_bf16 [8192, 2048]", "achieved": dom["gbps"],
                         "peak": PEAK_GBPS, "unit": "GB/s", "frac": dom["frac"],
                         "traffic": committed_traffic("norm_rows<unsigned short, 8, 1, 4, (Norm)1", 8192 * 64),
                         "algorithmic_bytes": dom["bytes"]},
        })
    if not args.no_cpu and head is not None:
        info_cpu = host_cpu()
        threads = info_cpu["affinity"]
        cpu = cpu_workloads(args.cpu_seconds / 6, threads)
        line["cpu_baseline"] = cpu_baseline(cpu, threads, info_cpu)
        for c, fig in cpu.items():
            if c in configs:
                configs[c]["cpu"] = {**fig, "threads": threads, "kind": "port"}
    line["configs"] = configs
    print(json.dumps(line), flush=True)
    reap_children()


def reap_children():
    """Ends the bench with no process of its own left behind: any child
    still alive (none is expected: workload 9's encoder runs under
    subprocess.run, which waits for it) is named on stderr, asked to end,
    then killed."""
    try:
        import psutil
    except ImportError:
        return
    kids = psutil.Process().children(recursive=True)
    for p in kids:
        try:
            print(f"[bench] child still running at exit: pid {p.pid} {' '.join(p.cmdline())}", file=sys.stderr,
                  flush=True)
            p.terminate()
        except psutil.Error:
            pass
    _, alive = psutil.wait_procs(kids, timeout=5)
    for p in alive:
        try:
            p.kill()
        except psutil.Error:
            pass


if __name__ == "__main__":
    main()
