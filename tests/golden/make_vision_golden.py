"""Writes tests/golden/vision_vectors.npz: small input/output vectors of the
vision encoder's ops produced by the reference's own CPU code
(src/backend/reference/ops.cpp: conv2d, layer_norm_channels, attention_head
with a bias, resize_bicubic_aa, resize_linear_rows, chw_to_hwc), compiled
from where it lies into oracle/_ref/libuocr_ref.so by `make -C oracle ref`.

Run in a container that holds the reference sources:
    make -C oracle ref && python tests/golden/make_vision_golden.py
The vectors let every machine check the oracle's restatement bit for bit
(tests/test_oracle_vision.py)."""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def main():
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libuocr_ref.so is not built: run `make -C oracle ref` first")
    p = lambda a: a.ctypes.data  # noqa: E731
    g = np.random.default_rng(20261202)
    f32 = lambda *s: g.standard_normal(s, dtype=np.float32)  # noqa: E731
    out = {}

    # the patch embedding's shape (kernel = stride) and a padded stride-2 3x3
    for tag, (c, h, w, o, k, stride, pad, bias) in {
        "patch": (3, 32, 32, 6, 8, 8, 0, True),
        "conv3": (5, 9, 9, 4, 3, 2, 1, False),
    }.items():
        x, wt = f32(c, h, w), 0.2 * f32(o, c, k, k)
        b = f32(o) if bias else None
        oh, ow = oracle.conv_out(h, k, stride, pad), oracle.conv_out(w, k, stride, pad)
        y = np.empty((o, oh, ow), np.float32)
        ref.ref_conv2d(p(x), c, h, w, p(wt), None if b is None else p(b), o, k, k, stride, pad, p(y))
        out.update({f"conv_{tag}_x": x, f"conv_{tag}_w": wt, f"conv_{tag}_y": y,
                    f"conv_{tag}_shape": np.array([stride, pad], np.int64)})
        if b is not None:
            out[f"conv_{tag}_b"] = b

    # channel LayerNorm over [c, h, w]
    x = 3 * f32(7, 5, 6) + 0.5
    lw, lb = (1 + 0.05 * f32(7)).astype(np.float32), 0.05 * f32(7)
    y = x.copy()
    ref.ref_layer_norm_channels(p(y), p(lw), p(lb), 7, 5, 6, np.float32(1e-6))
    out.update(lnc_x=x, lnc_w=lw, lnc_b=lb, lnc_y=y)

    # attention_head with a bias (the SAM form)
    q, k, v, bias = f32(11, 8), f32(13, 8), f32(13, 5), f32(11, 13)
    o = np.empty((11, 5), np.float32)
    ref.ref_attention_head(p(q), 11, p(k), 13, 8, p(v), 5, p(bias), np.float32(0.35), p(o))
    out.update(att_q=q, att_k=k, att_v=v, att_bias=bias, att_out=o)

    # bicubic antialiased resize: shrink (the SAM and CLIP position grids) and grow
    for tag, (c, h, w, oh, ow) in {"shrink": (3, 16, 16, 5, 5), "grow": (2, 4, 6, 9, 7)}.items():
        x = f32(c, h, w)
        y = np.empty((c, oh, ow), np.float32)
        ref.ref_resize_bicubic_aa(p(x), c, h, w, oh, ow, p(y))
        out.update({f"bicubic_{tag}_x": x, f"bicubic_{tag}_y": y})

    # linear row resize: the relative-position tables (127 -> 15 and 27 -> 53)
    for tag, (n, d, m) in {"shrink": (127, 6, 15), "grow": (27, 4, 53)}.items():
        x = f32(n, d)
        y = np.empty((m, d), np.float32)
        ref.ref_resize_linear_rows(p(x), n, d, m, p(y))
        out.update({f"linrows_{tag}_x": x, f"linrows_{tag}_y": y})

    np.savez_compressed(os.path.join(HERE, "vision_vectors.npz"), **out)
    print("wrote", os.path.join(HERE, "vision_vectors.npz"), sum(a.nbytes for a in out.values()), "bytes")


if __name__ == "__main__":
    main()
