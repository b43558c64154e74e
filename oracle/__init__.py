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
            "orc_chw_to_hwc": ([_vp, _i64, _i64, _i64, _vp], None),
            "orc_hwc_to_chw": ([_vp, _i64, _i64, _i64, _vp], None),
            "orc_concat_cols": ([_vp, _i64, _vp, _i64, _i64, _vp], None),
            "orc_im2col": ([_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp], None),
            "orc_conv2d": ([_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp], None),
            "orc_layer_norm_channels": ([_vp, _vp, _vp, _i64, _i64, _i64, _f], None),
            "orc_attention_head": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _f, _vp], None),
            "orc_resize_bicubic_aa": ([_vp, _i64, _i64, _i64, _i64, _i64, _vp], None),
            "orc_resize_linear_rows": ([_vp, _i64, _i64, _i64, _vp], None),
            "orc_relative_positions": ([_vp, _i64, _i64, _i64, _vp], None),
            "orc_rel_pos_bias": ([_vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp], None),
            "orc_page_image_tokens": ([_i64, _i64, _i64, _i64, ctypes.c_int], _i64),
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
            "ref_conv2d": ([_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp], None),
            "ref_layer_norm_channels": ([_vp, _vp, _vp, _i64, _i64, _i64, _f], None),
            "ref_resize_bicubic_aa": ([_vp, _i64, _i64, _i64, _i64, _i64, _vp], None),
            "ref_resize_linear_rows": ([_vp, _i64, _i64, _i64, _vp], None),
            "ref_chw_to_hwc": ([_vp, _i64, _i64, _i64, _vp], None),
            "ref_hwc_to_chw": ([_vp, _i64, _i64, _i64, _vp], None),
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


# ---- the vision encoder's ops (uocr_oracle_vision.c) -------------------------------------------


def chw_to_hwc(x) -> np.ndarray:
    """x [c, h, w] -> [h, w, c] (src/backend/reference/ops.cpp:298-304)."""
    x = _f32(x)
    c, h, w = x.shape
    y = np.empty((h, w, c), np.float32)
    lib().orc_chw_to_hwc(_p(x), c, h, w, _p(y))
    return y


def hwc_to_chw(x) -> np.ndarray:
    """x [h, w, c] -> [c, h, w] (ops.cpp:306-312)."""
    x = _f32(x)
    h, w, c = x.shape
    y = np.empty((c, h, w), np.float32)
    lib().orc_hwc_to_chw(_p(x), h, w, c, _p(y))
    return y


def concat_cols(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    rows = a.shape[0]
    out = np.empty((rows, a.shape[1] + b.shape[1]), np.float32)
    lib().orc_concat_cols(_p(a), a.shape[1], _p(b), b.shape[1], rows, _p(out))
    return out


def conv_out(size: int, k: int, stride: int, pad: int) -> int:
    return (size + 2 * pad - k) // stride + 1


def im2col(x, kh: int, kw: int, stride: int, pad: int) -> np.ndarray:
    """x [c, h, w] -> patches [oh * ow, c * kh * kw] (ops.cpp:198-212)."""
    x = _f32(x)
    c, h, w = x.shape
    oh, ow = conv_out(h, kh, stride, pad), conv_out(w, kw, stride, pad)
    cols = np.empty((oh * ow, c * kh * kw), np.float32)
    lib().orc_im2col(_p(x), c, h, w, kh, kw, stride, pad, _p(cols))
    return cols


def conv2d(x, weight, bias, stride: int, pad: int) -> np.ndarray:
    """x [c, h, w], weight [o, c, kh, kw] -> [o, oh, ow] (ops.cpp:189-217)."""
    x, wt = _f32(x), _f32(weight)
    b = None if bias is None else _f32(bias)
    c, h, w = x.shape
    o, _, kh, kw = wt.shape
    out = np.empty((o, conv_out(h, kh, stride, pad), conv_out(w, kw, stride, pad)), np.float32)
    lib().orc_conv2d(_p(x), c, h, w, _p(wt), _p(b), o, kh, kw, stride, pad, _p(out))
    return out


def layer_norm_channels(x, w, b, eps: float) -> np.ndarray:
    x, w, b = _f32(x), _f32(w), _f32(b)
    c, h, wd = x.shape
    lib().orc_layer_norm_channels(_p(x), _p(w), _p(b), c, h, wd, eps)
    return x


def attention_head(q, k, v, bias=None, scale: float = 1.0) -> np.ndarray:
    """q [lq, d], k [lk, d], v [lk, dv], bias [lq, lk] or None (ops.cpp:219-251)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b = None if bias is None else _f32(bias)
    lq, d = q.shape
    lk, dv = v.shape
    out = np.empty((lq, dv), np.float32)
    lib().orc_attention_head(_p(q), _p(k), _p(v), lq, lk, d, dv, _p(b), scale, _p(out))
    return out


def resize_bicubic_aa(x, oh: int, ow: int) -> np.ndarray:
    x = _f32(x)
    c, h, w = x.shape
    out = np.empty((c, oh, ow), np.float32)
    lib().orc_resize_bicubic_aa(_p(x), c, h, w, oh, ow, _p(out))
    return out


def resize_linear_rows(x, out_len: int) -> np.ndarray:
    x = _f32(x)
    n, c = x.shape
    out = np.empty((out_len, c), np.float32)
    lib().orc_resize_linear_rows(_p(x), n, c, out_len, _p(out))
    return out


def relative_positions(table, size: int) -> np.ndarray:
    """[size, size, d]: entry [q][k] = the table (resized to 2 size - 1 rows)
    at row q - k + size - 1 (src/model/sam_encoder.cpp:52-63)."""
    t = _f32(table)
    n, d = t.shape
    out = np.empty((size, size, d), np.float32)
    lib().orc_relative_positions(_p(t), n, d, size, _p(out))
    return out


def rel_pos_bias(q, h: int, w: int, rh, rw) -> np.ndarray:
    """q [h * w, d] (rows may be wider: only the first d columns of rh's
    width are read), rh [h, h, d], rw [w, w, d] -> bias [h * w, h * w]."""
    q, rh, rw = _f32(q), _f32(rh), _f32(rw)
    d = rh.shape[-1]
    out = np.empty((h * w, h * w), np.float32)
    lib().orc_rel_pos_bias(_p(q), q.shape[1], h, w, d, _p(rh), _p(rw), _p(out))
    return out


def page_image_tokens(global_grid: int, tile_grid: int, tiles_wide: int, tiles_high: int, tiled: bool) -> int:
    return int(lib().orc_page_image_tokens(global_grid, tile_grid, tiles_wide, tiles_high, int(tiled)))


# ---- the vision encoder (uocr_oracle_vision.c: orc_encode_view / orc_encode_page) ---------------

class _SamDims(ctypes.Structure):
    _fields_ = [(n, _i64) for n in ("image", "patch", "width", "layers", "heads", "mlp", "window", "neck", "net2",
                                     "net3")]


class _SamBlock(ctypes.Structure):
    _fields_ = ([(n, _vp) for n in ("norm1_w", "norm1_b", "qkv_w", "qkv_b", "proj_w", "proj_b", "rel_h", "rel_w")]
                + [("rel_len", _i64)]
                + [(n, _vp) for n in ("norm2_w", "norm2_b", "lin1_w", "lin1_b", "lin2_w", "lin2_b")]
                + [("global_", ctypes.c_int)])


class _SamWeights(ctypes.Structure):
    _fields_ = [(n, _vp) for n in ("patch_w", "patch_b", "pos_embed", "blocks", "neck0_w", "neck1_w", "neck1_b",
                                    "neck2_w", "neck3_w", "neck3_b", "net2_w", "net3_w")]


class _ClipDims(ctypes.Structure):
    _fields_ = [(n, _i64) for n in ("width", "layers", "heads", "mlp", "positions")]


class _ClipLayer(ctypes.Structure):
    _fields_ = [(n, _vp) for n in ("ln1_w", "ln1_b", "qkv_w", "qkv_b", "out_w", "out_b", "ln2_w", "ln2_b", "fc1_w",
                                    "fc1_b", "fc2_w", "fc2_b")]


class _ClipWeights(ctypes.Structure):
    _fields_ = [(n, _vp) for n in ("class_embedding", "positions", "pre_ln_w", "pre_ln_b", "layers")]


class _VisionWeights(ctypes.Structure):
    _fields_ = [("sam_dims", _SamDims), ("sam", _SamWeights), ("clip_dims", _ClipDims), ("clip", _ClipWeights),
                ("projector_w", _vp), ("projector_b", _vp), ("newline", _vp), ("separator", _vp),
                ("hidden", _i64)]


class VisionModel:
    """The reference's vision encoder over a dict of fp32 tensors named as
    in the checkpoint (src/weights/architecture.cpp:38-85,137-139), dims as
    SamDims / ClipDims (src/weights/architecture.h:35-56) plus `hidden`.
    round_x rounds every linear's input to bf16 as the device linear does."""

    SAM = "model.sam_model"
    CLIP = "model.vision_model"

    def __init__(self, weights: dict, sam: dict, clip: dict, hidden: int):
        self.w = {k: _f32(v) for k, v in weights.items()}
        self.sam, self.clip, self.hidden = dict(sam), dict(clip), hidden
        g = lambda name: _p(self.w[name])  # noqa: E731
        s, c = self.SAM, self.CLIP
        self._blocks = (_SamBlock * sam["layers"])()
        for i in range(sam["layers"]):
            p = f"{s}.blocks.{i}."
            b = self._blocks[i]
            for f, n in (("norm1_w", "norm1.weight"), ("norm1_b", "norm1.bias"), ("qkv_w", "attn.qkv.weight"),
                         ("qkv_b", "attn.qkv.bias"), ("proj_w", "attn.proj.weight"), ("proj_b", "attn.proj.bias"),
                         ("rel_h", "attn.rel_pos_h"), ("rel_w", "attn.rel_pos_w"), ("norm2_w", "norm2.weight"),
                         ("norm2_b", "norm2.bias"), ("lin1_w", "mlp.lin1.weight"), ("lin1_b", "mlp.lin1.bias"),
                         ("lin2_w", "mlp.lin2.weight"), ("lin2_b", "mlp.lin2.bias")):
                setattr(b, f, g(p + n))
            b.rel_len = self.w[p + "attn.rel_pos_h"].shape[0]
            b.global_ = int(i in sam["global_layers"])
        self._layers = (_ClipLayer * clip["layers"])()
        for i in range(clip["layers"]):
            p = f"{c}.transformer.layers.{i}."
            l = self._layers[i]
            for f, n in (("ln1_w", "layer_norm1.weight"), ("ln1_b", "layer_norm1.bias"),
                         ("qkv_w", "self_attn.qkv_proj.weight"), ("qkv_b", "self_attn.qkv_proj.bias"),
                         ("out_w", "self_attn.out_proj.weight"), ("out_b", "self_attn.out_proj.bias"),
                         ("ln2_w", "layer_norm2.weight"), ("ln2_b", "layer_norm2.bias"),
                         ("fc1_w", "mlp.fc1.weight"), ("fc1_b", "mlp.fc1.bias"), ("fc2_w", "mlp.fc2.weight"),
                         ("fc2_b", "mlp.fc2.bias")):
                setattr(l, f, g(p + n))
        vw = _VisionWeights()
        vw.sam_dims = _SamDims(*[sam[n] for n in ("image", "patch", "width", "layers", "heads", "mlp", "window",
                                                  "neck", "net2", "net3")])
        vw.sam = _SamWeights(g(s + ".patch_embed.proj.weight"), g(s + ".patch_embed.proj.bias"), g(s + ".pos_embed"),
                             ctypes.cast(self._blocks, _vp), g(s + ".neck.0.weight"), g(s + ".neck.1.weight"),
                             g(s + ".neck.1.bias"), g(s + ".neck.2.weight"), g(s + ".neck.3.weight"),
                             g(s + ".neck.3.bias"), g(s + ".net_2.weight"), g(s + ".net_3.weight"))
        vw.clip_dims = _ClipDims(clip["width"], clip["layers"], clip["heads"], clip["mlp"], clip["positions"])
        vw.clip = _ClipWeights(g(c + ".embeddings.class_embedding"), g(c + ".embeddings.position_embedding.weight"),
                               g(c + ".pre_layrnorm.weight"), g(c + ".pre_layrnorm.bias"),
                               ctypes.cast(self._layers, _vp))
        vw.projector_w, vw.projector_b = g("model.projector.layers.weight"), g("model.projector.layers.bias")
        vw.newline, vw.separator = g("model.image_newline"), g("model.view_seperator")
        vw.hidden = hidden
        self._vw = vw
        h = lib()
        for name, args, res in (
                ("orc_encode_view", [_vp, _vp, _i64, _vp, ctypes.c_int], _i64),
                ("orc_encode_page", [_vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, ctypes.c_int], _i64)):
            getattr(h, name).argtypes = args
            getattr(h, name).restype = res

    def grid(self, size: int) -> int:
        g = size // self.sam["patch"]
        return conv_out(conv_out(g, 3, 2, 1), 3, 2, 1)

    def encode_view(self, image, round_x: bool = False) -> np.ndarray:
        img = _f32(image)
        s = img.shape[1]
        g = self.grid(s)
        out = np.empty((g * g, self.hidden), np.float32)
        got = lib().orc_encode_view(ctypes.byref(self._vw), _p(img), s, _p(out), int(round_x))
        if got != g:
            raise ValueError("encode_view: bad image shape")
        return out

    def encode_page(self, global_image, tiles=(), tiles_wide: int = 1, tiles_high: int = 1,
                    round_x: bool = False) -> np.ndarray:
        gi = _f32(global_image)
        gs = gi.shape[1]
        t = _f32(np.stack(tiles)) if len(tiles) else np.zeros(1, np.float32)
        ts = t.shape[2] if len(tiles) else 0
        rows = page_image_tokens(self.grid(gs), self.grid(ts) if ts else 0, tiles_wide, tiles_high, len(tiles) > 0)
        out = np.empty((rows, self.hidden), np.float32)
        got = lib().orc_encode_page(ctypes.byref(self._vw), _p(gi), gs, _p(t), len(tiles), ts, tiles_wide,
                                    tiles_high, _p(out), int(round_x))
        if got != rows:
            raise ValueError("encode_page: bad shapes")
        return out


def vision_tensor_shapes(sam: dict, clip: dict, hidden: int) -> dict:
    """The vision tensors' shapes as the reference's architecture table
    lists them (src/weights/architecture.cpp:38-85,137-139)."""
    s, c = VisionModel.SAM, VisionModel.CLIP
    grid, hd = sam["image"] // sam["patch"], sam["width"] // sam["heads"]
    out = {s + ".patch_embed.proj.weight": (sam["width"], 3, sam["patch"], sam["patch"]),
           s + ".patch_embed.proj.bias": (sam["width"],), s + ".pos_embed": (1, grid, grid, sam["width"])}
    for i in range(sam["layers"]):
        p = f"{s}.blocks.{i}."
        span = grid if i in sam["global_layers"] else sam["window"]
        out.update({p + "norm1.weight": (sam["width"],), p + "norm1.bias": (sam["width"],),
                    p + "attn.qkv.weight": (3 * sam["width"], sam["width"]), p + "attn.qkv.bias": (3 * sam["width"],),
                    p + "attn.proj.weight": (sam["width"], sam["width"]), p + "attn.proj.bias": (sam["width"],),
                    p + "attn.rel_pos_h": (2 * span - 1, hd), p + "attn.rel_pos_w": (2 * span - 1, hd),
                    p + "norm2.weight": (sam["width"],), p + "norm2.bias": (sam["width"],),
                    p + "mlp.lin1.weight": (sam["mlp"], sam["width"]), p + "mlp.lin1.bias": (sam["mlp"],),
                    p + "mlp.lin2.weight": (sam["width"], sam["mlp"]), p + "mlp.lin2.bias": (sam["width"],)})
    out.update({s + ".neck.0.weight": (sam["neck"], sam["width"], 1, 1), s + ".neck.1.weight": (sam["neck"],),
                s + ".neck.1.bias": (sam["neck"],), s + ".neck.2.weight": (sam["neck"], sam["neck"], 3, 3),
                s + ".neck.3.weight": (sam["neck"],), s + ".neck.3.bias": (sam["neck"],),
                s + ".net_2.weight": (sam["net2"], sam["neck"], 3, 3),
                s + ".net_3.weight": (sam["net3"], sam["net2"], 3, 3)})
    out.update({c + ".embeddings.class_embedding": (clip["width"],),
                c + ".embeddings.position_embedding.weight": (clip["positions"], clip["width"]),
                c + ".pre_layrnorm.weight": (clip["width"],), c + ".pre_layrnorm.bias": (clip["width"],)})
    for i in range(clip["layers"]):
        p = f"{c}.transformer.layers.{i}."
        w = clip["width"]
        out.update({p + "layer_norm1.weight": (w,), p + "layer_norm1.bias": (w,),
                    p + "self_attn.qkv_proj.weight": (3 * w, w), p + "self_attn.qkv_proj.bias": (3 * w,),
                    p + "self_attn.out_proj.weight": (w, w), p + "self_attn.out_proj.bias": (w,),
                    p + "layer_norm2.weight": (w,), p + "layer_norm2.bias": (w,),
                    p + "mlp.fc1.weight": (clip["mlp"], w), p + "mlp.fc1.bias": (clip["mlp"],),
                    p + "mlp.fc2.weight": (w, clip["mlp"]), p + "mlp.fc2.bias": (w,)})
    out.update({"model.projector.layers.weight": (hidden, clip["width"] + sam["net3"]),
                "model.projector.layers.bias": (hidden,), "model.image_newline": (hidden,),
                "model.view_seperator": (hidden,)})
    return out


TINY_SAM = dict(image=1024, patch=16, width=24, layers=2, heads=2, mlp=48, window=14, global_layers=(1,), neck=8,
                net2=12, net3=16)
TINY_CLIP = dict(width=16, layers=2, heads=2, mlp=32, positions=257)
TINY_HIDDEN = 20


def tiny_vision_weights(seed: int = 7, bf16_grid: bool = True) -> dict:
    """Random parameters for the reference's tiny test model
    (tests/cuda_vision_test.cpp:33-51): N(0, 0.05), norm weights 1 + N(0,
    0.05), on the bf16 grid so the device and the oracle see the same values."""
    g = np.random.default_rng(seed)
    out = {}
    for name, shape in vision_tensor_shapes(TINY_SAM, TINY_CLIP, TINY_HIDDEN).items():
        v = 0.05 * g.standard_normal(shape).astype(np.float32)
        if "norm" in name and name.endswith(".weight"):
            v = v + 1.0
        out[name] = bf16_round(v) if bf16_grid else v.astype(np.float32)
    return out
