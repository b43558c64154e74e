"""numpy wrappers over the CPU oracle (oracle/uocr_oracle.c) and, where it was
built, over the reference's own CPU ops (oracle/_ref/libuocr_ref.so).

TEST INFRASTRUCTURE ONLY. Imported by tests/, by __graft_entry__.smoke() to
check its result, and by bench.py's cpu_baseline leg to time the reference's
CPU path. It is never part of a product path: the ops themselves are the HIP
library in grpc-unlimited-ocr_amd/.

Every wrapper copies its inputs and returns new arrays; float32 in, float32
out, bf16 as uint16 bits. The C functions each cite the reference file:line
they restate.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libuocr_ref.so")

_LIB = None
_REF = None

_f = ctypes.c_float
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


def build() -> None:
    """Compile the oracle (and oracle/_ref when the reference sources exist)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-s", "-C", HERE], check=True)
        h = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_bf16_to_f32": ([ctypes.c_uint16], _f),
            "orc_f32_to_bf16": ([_f], ctypes.c_uint16),
            "orc_f32_to_bf16_array": ([_vp, _vp, _i64], None),
            "orc_bf16_to_f32_array": ([_vp, _vp, _i64], None),
            "orc_set_threads": ([ctypes.c_int], None),
            "orc_threads": ([], ctypes.c_int),
            "orc_rms_norm": ([_vp, _vp, _i64, _i64, _f], None),
            "orc_layer_norm": ([_vp, _vp, _vp, _i64, _i64, _f], None),
            "orc_gelu_erf": ([_vp, _i64], None),
            "orc_silu": ([_vp, _i64], None),
            "orc_mul_into": ([_vp, _vp, _i64], None),
            "orc_add_into": ([_vp, _vp, _i64], None),
            "orc_rope_inv": ([_vp, _i64, ctypes.c_double], None),
            "orc_rope_apply": ([_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64], None),
            "orc_embed": ([_vp, _vp, _i64, _i64, _vp], None),
            "orc_add_rms_norm": ([_vp, _vp, _vp, _vp, _i64, _i64, _f], None),
            "orc_decode_chain": ([_vp, _i64, _vp, _vp, _vp, _vp, _i64, _f, _vp, _i64, _vp, _i64, _i64, _i64, _vp,
                                  _i64, _i64], None),
            "orc_swiglu": ([_vp, _vp, _i64, _i64], None),
            "orc_router_norm": ([_vp, _vp, _i64, _i64, _f], None),
            "orc_linear": ([_vp, _i64, _i64, _vp, _i64, _vp, _vp], None),
            "orc_softmax_rows": ([_vp, _i64, _i64], None),
            "orc_attention_one": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _f, _vp], None),
            "orc_scale_add_mask": ([_vp, _f, _vp, _i64, _i64, _i64], None),
            "orc_quick_gelu": ([_vp, _i64], None),
            "orc_expert_topk": ([_vp, _i64, _i64, _i64, _vp, _vp], None),
            "orc_block_summaries": ([_vp, _i64, _i64, _vp, _i64, _vp], None),
            "orc_block_scores": ([_vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp], None),
            "orc_entmax15": ([_vp, _i64], None),
            "orc_select_blocks": ([_vp, _i64, _i64, _vp, _i64, _i64, _f, _f, _f, _vp, _vp, _vp], _i64),
            "orc_key_mask": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp], None),
            "orc_page_candidates": ([_vp, _vp, _i64, _i64, _i64, _vp], ctypes.c_int),
            "orc_route_one": ([_vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f, _f,
                               _f, _vp, _vp], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = h
    return _LIB


def ref_lib() -> Optional[ctypes.CDLL]:
    """The reference's own CPU ops, or None where oracle/_ref was not built."""
    global _REF
    if _REF is None and os.path.exists(REF_LIB_PATH):
        h = ctypes.CDLL(REF_LIB_PATH)
        sig = {
            "ref_set_threads": ([ctypes.c_uint], None),
            "ref_f32_to_bf16": ([_f], ctypes.c_uint16),
            "ref_bf16_to_f32": ([ctypes.c_uint16], _f),
            "ref_rms_norm": ([_vp, _vp, _i64, _i64, _f], None),
            "ref_layer_norm": ([_vp, _vp, _vp, _i64, _i64, _f], None),
            "ref_gelu_erf": ([_vp, _i64], None),
            "ref_silu": ([_vp, _i64], None),
            "ref_rope_tables": ([_i64, ctypes.c_double, ctypes.c_double, _i64, _vp, _vp], None),
            "ref_rope_apply": ([_vp, _i64, _i64, _i64, ctypes.c_double, ctypes.c_double, _i64, _i64, _vp, _vp],
                               None),
            "ref_quick_gelu": ([_vp, _i64], None),
            "ref_softmax_rows": ([_vp, _i64, _i64], None),
            "ref_linear": ([_vp, _i64, _i64, _vp, _i64, _vp, _vp], None),
            "ref_attention_head": ([_vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _f, _vp], None),
            "ref_block_summaries": ([_vp, _i64, _i64, _vp, _i64, _vp], None),
            "ref_block_scores": ([_vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp], None),
            "ref_entmax15": ([_vp, _i64], None),
            "ref_select_blocks": ([_vp, _i64, _i64, _vp, _i64, _i64, _f, _f, _f, _vp, _vp, _vp], _i64),
            "ref_key_mask": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = res
        _REF = h
    return _REF


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).copy()


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


# ---- bf16 ---------------------------------------------------------------------


def f32_to_bf16(a) -> np.ndarray:
    a = _f32(a)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_array(_p(a), _p(out), a.size)
    return out


def bf16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().orc_bf16_to_f32_array(_p(b), _p(out), b.size)
    return out


def bf16_round(a) -> np.ndarray:
    """float32 values rounded to the bf16 grid (nearest even)."""
    return bf16_to_f32(f32_to_bf16(a))


# ---- threading ------------------------------------------------------------------


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def threads() -> int:
    return lib().orc_threads()


# ---- ops --------------------------------------------------------------------------


def rms_norm(x, w, eps: float) -> np.ndarray:
    x = _f32(x)
    w = _f32(w)
    cols = x.shape[-1]
    lib().orc_rms_norm(_p(x), _p(w), x.size // cols, cols, eps)
    return x


def layer_norm(x, w, b, eps: float) -> np.ndarray:
    x = _f32(x)
    w, b = _f32(w), _f32(b)
    cols = x.shape[-1]
    lib().orc_layer_norm(_p(x), _p(w), _p(b), x.size // cols, cols, eps)
    return x


def gelu_erf(x) -> np.ndarray:
    x = _f32(x)
    lib().orc_gelu_erf(_p(x), x.size)
    return x


def silu(x) -> np.ndarray:
    x = _f32(x)
    lib().orc_silu(_p(x), x.size)
    return x


def silu_mul(g, u) -> np.ndarray:
    g = silu(g)
    u = _f32(u)
    lib().orc_mul_into(_p(g), _p(u), g.size)
    return g


def add(x, y) -> np.ndarray:
    x = _f32(x)
    y = _f32(y)
    lib().orc_add_into(_p(x), _p(y), x.size)
    return x


def add_rms_norm(x, delta, w, eps: float):
    """(x + delta, rms_norm(x + delta) * w), the reference's add/copy/norm chain."""
    x = _f32(x)
    d, w = _f32(delta), _f32(w)
    h = np.empty_like(x)
    cols = x.shape[-1]
    lib().orc_add_rms_norm(_p(x), _p(d), _p(w), _p(h), x.size // cols, cols, eps)
    return x, h


def swiglu(inp) -> np.ndarray:
    inp = _f32(inp)
    two_f = inp.shape[-1]
    rows, ffn = inp.size // two_f, two_f // 2
    out = np.empty(inp.shape[:-1] + (ffn,), dtype=np.float32)
    lib().orc_swiglu(_p(inp), _p(out), rows, ffn)
    return out


def rope_inv(n: int, theta: float) -> np.ndarray:
    inv = np.empty(n, dtype=np.float32)
    lib().orc_rope_inv(_p(inv), n, theta)
    return inv


def rope(x, heads: int, dim: int, tok=None, page=None, inv_tok=None, inv_page=None, page_mod: int = 0,
         one_tok: int = 0, one_page: int = 0) -> np.ndarray:
    x = _f32(x)
    rows = x.size // (heads * dim)
    tok = None if tok is None else np.ascontiguousarray(tok, dtype=np.int64)
    page = None if page is None else np.ascontiguousarray(page, dtype=np.int64)
    inv_tok = np.zeros(0, np.float32) if inv_tok is None else _f32(inv_tok)
    inv_page = np.zeros(0, np.float32) if inv_page is None else _f32(inv_page)
    lib().orc_rope_apply(_p(x), rows, heads, dim, _p(tok), _p(page), _p(inv_tok), inv_tok.size, _p(inv_page),
                         inv_page.size, page_mod, one_tok, one_page)
    return x


def embed(table_bits, ids) -> np.ndarray:
    table_bits = np.ascontiguousarray(table_bits, dtype=np.uint16)
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    cols = table_bits.shape[-1]
    out = np.empty((ids.size, cols), dtype=np.float32)
    lib().orc_embed(_p(table_bits), _p(ids), ids.size, cols, _p(out))
    return out


# ---- the decode-step neighbours and the row ops beside the path ---------------------------------


def router_norm(x, w, eps: float) -> np.ndarray:
    x = _f32(x)
    w = _f32(w)
    cols = x.shape[-1]
    lib().orc_router_norm(_p(x), _p(w), x.size // cols, cols, eps)
    return x


def linear(x, w, bias=None) -> np.ndarray:
    """x [m, k] times w [n, k] transposed (+ bias [n]): [m, n]."""
    x = _f32(np.atleast_2d(x))
    w = _f32(w)
    b = None if bias is None else _f32(bias)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    lib().orc_linear(_p(x), m, k, _p(w), n, _p(b), _p(y))
    return y


def softmax_rows(x) -> np.ndarray:
    x = _f32(x)
    cols = x.shape[-1]
    lib().orc_softmax_rows(_p(x), x.size // cols, cols)
    return x


def expert_topk(logits, k: int):
    """Softmax over each row of gate logits [rows, experts], then the k top
    scores, lower index first on a tie (src/model/feed_forward.cpp:36-53):
    (ids int64 [rows, k], weights float32 [rows, k])."""
    x = _f32(logits)
    experts = x.shape[-1]
    rows = x.size // experts
    ids = np.empty((rows, k), np.int64)
    w = np.empty((rows, k), np.float32)
    lib().orc_expert_topk(_p(x), rows, experts, k, _p(ids), _p(w))
    return ids, w


def attention_one(q, k, v, heads: int, hd: int, bias=None, scale: float = 1.0) -> np.ndarray:
    """One query per head over keys [keys, heads * hd] with an optional
    [keys] additive mask shared by the heads: [heads * hd]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    keys = k.shape[0]
    b = None if bias is None else _f32(bias)
    out = np.empty(heads * hd, np.float32)
    lib().orc_attention_one(_p(q), _p(k), _p(v), keys, heads * hd, heads, hd, _p(b), scale, _p(out))
    return out


def scale_add_mask(x, scale: float, mask, batch: int, rows: int, cols: int) -> np.ndarray:
    x = _f32(x)
    m = None if mask is None else _f32(mask)
    lib().orc_scale_add_mask(_p(x), scale, _p(m), batch, rows, cols)
    return x


def quick_gelu(x) -> np.ndarray:
    x = _f32(x)
    lib().orc_quick_gelu(_p(x), x.size)
    return x


# ---- the block router (src/model/block_router.cpp, attention_plan.cpp) -----------------------


class RouterParams:
    """The reference's RouterParams (src/model/block_router.h:16-26) with
    Decoder::default_router's idx_scale (src/model/decoder.cpp:58-62)."""

    def __init__(self, block_size=32, local_blocks=4, top_m=16, top_k=12, idx_scale=None, floor=1e-4, sigma=1.0):
        self.block_size, self.local_blocks, self.top_m, self.top_k = block_size, local_blocks, top_m, top_k
        self.idx_scale = float(np.float32(128.0) / np.sqrt(np.float32(128.0))) if idx_scale is None else idx_scale
        self.floor, self.sigma = floor, sigma


def block_summaries(rk, cls, block_size: int) -> np.ndarray:
    rk, cls = _f32(rk), _f32(cls)
    keys, d = rk.shape
    out = np.empty(((keys + block_size - 1) // block_size, d), np.float32)
    lib().orc_block_summaries(_p(rk), keys, d, _p(cls), block_size, _p(out))
    return out


def block_scores(rq, summaries, q_pos, block_size: int, local_blocks: int) -> np.ndarray:
    rq, summaries = _f32(rq).reshape(-1, _f32(summaries).shape[1]), _f32(summaries)
    q_pos = np.ascontiguousarray(q_pos, dtype=np.int64)
    out = np.empty((rq.shape[0], summaries.shape[0]), np.float32)
    lib().orc_block_scores(_p(rq), rq.shape[0], _p(summaries), summaries.shape[0], summaries.shape[1], _p(q_pos),
                           block_size, local_blocks, _p(out))
    return out


def entmax15(x) -> np.ndarray:
    x = _f32(x)
    lib().orc_entmax15(_p(x), x.size)
    return x


def select_blocks(scores, candidate, p: RouterParams):
    """(block, bias, valid) [lq, width] of each score row."""
    scores = _f32(scores)
    lq, nblk = scores.shape
    cand = None if candidate is None else np.ascontiguousarray(candidate, dtype=np.uint8)
    cap = max(1, p.top_k)
    block, bias, valid = np.empty(lq * cap, np.int64), np.empty(lq * cap, np.float32), np.empty(lq * cap, np.uint8)
    w = lib().orc_select_blocks(_p(scores), lq, nblk, _p(cand), p.top_m, p.top_k, p.idx_scale, p.floor, p.sigma,
                                _p(block), _p(bias), _p(valid))
    return block[:lq * w].reshape(lq, w), bias[:lq * w].reshape(lq, w), valid[:lq * w].reshape(lq, w)


def key_mask(block, bias, valid, first_pos: int, keys: int, p: RouterParams) -> np.ndarray:
    block = np.ascontiguousarray(block, dtype=np.int64)
    bias, valid = _f32(bias), np.ascontiguousarray(valid, dtype=np.uint8)
    rows, width = block.shape
    out = np.empty((rows, keys), np.float32)
    lib().orc_key_mask(_p(block), _p(bias), _p(valid), width, rows, first_pos, keys, p.block_size, p.local_blocks,
                       _p(out))
    return out


def page_candidates(min_page, max_page, page: int, nblk: int):
    """[nblk] uint8, or None for no restriction."""
    lo = np.ascontiguousarray(min_page, dtype=np.int64)
    hi = np.ascontiguousarray(max_page, dtype=np.int64)
    out = np.zeros(max(1, nblk), np.uint8)
    any_ = lib().orc_page_candidates(_p(lo), _p(hi), lo.size, page, nblk, _p(out))
    return out[:nblk] if any_ else None


def route_one(rq, rk, pos: int, cls, p: RouterParams, min_page=None, max_page=None, query_page: int = -1):
    """(summaries, mask [pos + 1]) of one decode query over router keys rk [pos + 1, d]."""
    rq, rk, cls = _f32(rq), _f32(rk), _f32(cls)
    d = rq.size
    lo = np.zeros(1, np.int64) if min_page is None else np.ascontiguousarray(min_page, dtype=np.int64)
    hi = np.zeros(1, np.int64) if max_page is None else np.ascontiguousarray(max_page, dtype=np.int64)
    known = 0 if min_page is None else lo.size
    summaries = np.empty(((pos + 1 + p.block_size - 1) // p.block_size, d), np.float32)
    mask = np.empty(pos + 1, np.float32)
    lib().orc_route_one(_p(rq), _p(rk), pos, d, _p(cls), _p(lo), _p(hi), known, query_page, p.block_size,
                        p.local_blocks, p.top_m, p.top_k, p.idx_scale, p.floor, p.sigma, _p(summaries), _p(mask))
    return summaries, mask
