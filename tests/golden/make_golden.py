"""Writes tests/golden/ref_vectors.npz: small input/output vectors produced by
the reference's own CPU code (src/backend/reference/ops.cpp,
src/model/page_rope.cpp, src/model/block_router.cpp,
src/model/attention_plan.cpp, src/tensor/dtype.h), compiled from where it lies
into oracle/_ref/libuocr_ref.so by `make -C oracle ref`.

Run in a container that holds the reference sources:
    make -C oracle ref && python tests/golden/make_golden.py
The vectors let every machine (including ones without the reference) check
the oracle's restatement bit for bit (tests/test_oracle.py)."""

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
    g = np.random.default_rng(20260101)
    out = {}

    # norms: [6, 300] like the reference's device test, eps 1e-6
    x = g.standard_normal((6, 300), dtype=np.float32) * 2 + 0.5
    w = (1 + 0.02 * g.standard_normal(300)).astype(np.float32)
    b = (0.02 * g.standard_normal(300)).astype(np.float32)
    r = x.copy()
    ref.ref_rms_norm(p(r), p(w), 6, 300, np.float32(1e-6))
    l = x.copy()
    ref.ref_layer_norm(p(l), p(w), p(b), 6, 300, np.float32(1e-6))
    out.update(norm_x=x, norm_w=w, norm_b=b, norm_eps=np.float32(1e-6), rms_out=r, ln_out=l)

    # activations over a spread that reaches the tails
    a = (g.standard_normal(2048) * 4).astype(np.float32)
    ge, si = a.copy(), a.copy()
    ref.ref_gelu_erf(p(ge), ge.size)
    ref.ref_silu(p(si), si.size)
    out.update(act_x=a, gelu_out=ge, silu_out=si)

    # the decoder's two-axis rope: dim 128, 63 token pairs + 1 page pair, page mod 2
    dim, heads, pairs, rows = 128, 3, 1, 8
    inv_tok = np.empty(dim // 2 - pairs, np.float32)
    inv_page = np.empty(pairs, np.float32)
    ref.ref_rope_tables(dim, 1e4, 256.0, pairs, p(inv_tok), p(inv_page))
    xr = g.standard_normal((rows, heads * dim), dtype=np.float32)
    tok = np.array([0, 1, 17, 300, 4095, 8191, 12000, 20000], np.int64)
    page = np.array([0, 1, 2, 3, -1, 7, 10, 11], np.int64)
    yr = xr.copy()
    ref.ref_rope_apply(p(yr), rows, heads * dim, dim, 1e4, 256.0, pairs, 2, p(tok), p(page))
    out.update(rope_x=xr, rope_out=yr, rope_tok=tok, rope_page=page, rope_inv_tok=inv_tok, rope_inv_page=inv_page,
               rope_dim=np.int64(dim), rope_heads=np.int64(heads), rope_page_mod=np.int64(2),
               rope_tok_theta=np.float64(1e4), rope_page_theta=np.float64(256.0))

    # bf16 rounding: ties, near-ties, overflow, NaN, and random patterns
    special = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0x7F7FFFFF, 0x7F7F8000, 0xFF7F8000, 0x7FC00001,
                        0xFFA00000, 0x00008000, 0x00018000, 0x80008000, 0x7F800000, 0x00000001], np.uint32)
    bits = np.concatenate([special, g.integers(0, 1 << 32, 2048, dtype=np.uint64).astype(np.uint32)])
    bf = np.array([ref.ref_f32_to_bf16(np.float32(v)) for v in bits.view(np.float32)], np.uint16)
    out.update(bf16_in=bits, bf16_out=bf)

    # the ops beside the path: softmax_rows, linear, attention_head, quick_gelu
    sm = (g.standard_normal((5, 333)) * 3).astype(np.float32)
    sm[2, :] = -np.inf
    sm[3, ::3] = -np.inf
    smo = sm.copy()
    ref.ref_softmax_rows(p(smo), 5, 333)
    lx = g.standard_normal((3, 200), dtype=np.float32)
    lw = (g.standard_normal((7, 200)) * 0.1).astype(np.float32)
    lb = g.standard_normal(7, dtype=np.float32)
    ly = np.empty((3, 7), np.float32)
    ref.ref_linear(p(lx), 3, 200, p(lw), 7, p(lb), p(ly))
    aq = g.standard_normal((1, 64), dtype=np.float32)
    ak = g.standard_normal((50, 64), dtype=np.float32)
    av = g.standard_normal((50, 64), dtype=np.float32)
    am = np.zeros((1, 50), np.float32)
    am[0, 10:30] = -np.inf
    ao = np.empty((1, 64), np.float32)
    ref.ref_attention_head(p(aq), 1, p(ak), 50, 64, p(av), 64, p(am), np.float32(0.125), p(ao))
    qg = a.copy()
    ref.ref_quick_gelu(p(qg), qg.size)
    out.update(softmax_in=sm, softmax_out=smo, linear_x=lx, linear_w=lw, linear_b=lb, linear_y=ly,
               attn_q=aq, attn_k=ak, attn_v=av, attn_mask=am, attn_scale=np.float32(0.125), attn_out=ao,
               quick_gelu_out=qg)

    # the block router: summaries, scores, selection (with candidates), key mask, entmax
    d, keys = 64, 300
    rk = (g.standard_normal((keys, d)) * 2).astype(np.float32)
    cls = g.standard_normal(d, dtype=np.float32)
    nblk = (keys + 31) // 32
    summ = np.empty((nblk, d), np.float32)
    ref.ref_block_summaries(p(rk), keys, d, p(cls), 32, p(summ))
    rq = g.standard_normal((4, d), dtype=np.float32)
    qpos = np.array([keys - 4, keys - 3, keys - 2, keys - 1], np.int64)
    sc = np.empty((4, nblk), np.float32)
    ref.ref_block_scores(p(rq), 4, p(summ), nblk, d, p(qpos), 32, 4, p(sc))
    cand = (g.random((4, nblk)) < 0.4).astype(np.uint8)
    cand[3] = 0  # a row whose candidates exclude every remote block
    prm = oracle.RouterParams()
    blk, bia, val = np.empty(4 * 12, np.int64), np.empty(4 * 12, np.float32), np.empty(4 * 12, np.uint8)
    wid = ref.ref_select_blocks(p(sc), 4, nblk, p(cand), prm.top_m, prm.top_k, np.float32(prm.idx_scale),
                                np.float32(prm.floor), np.float32(prm.sigma), p(blk), p(bia), p(val))
    blk, bia, val = blk[:4 * wid].reshape(4, wid), bia[:4 * wid].reshape(4, wid), val[:4 * wid].reshape(4, wid)
    msk = np.empty((4, keys), np.float32)
    ref.ref_key_mask(p(blk), p(bia), p(val), wid, 4, keys - 4, keys, 32, 4, p(msk))
    ei = (g.standard_normal(16) * 3).astype(np.float32)
    eo = ei.copy()
    ref.ref_entmax15(p(eo), 16)
    out.update(router_rk=rk, router_cls=cls, router_summaries=summ, router_rq=rq, router_pos=qpos, router_scores=sc,
               router_cand=cand, router_block=blk, router_bias=bia, router_valid=val, router_first=np.int64(keys - 4),
               router_keys=np.int64(keys), router_mask=msk, entmax_in=ei, entmax_out=eo)

    path = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
