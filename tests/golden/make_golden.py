"""Write tests/golden/jasmine_golden.npz from the jasmine reference itself.

Runs only where oracle/_ref/libjasref.so was built (it compiles the reference's own
headers; see oracle/Makefile).  Every array is an input or an output of a reference call
on small seeded inputs; nothing else is stored.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from oracle_lib import ref, normal, fp, ip  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "jasmine_golden.npz")

# (id, a_shape, b_shape) for ref_expr; b shapes exercise jasmine's modulo broadcasting
EXPR_CASES = [
    (0, (5, 7), (5, 7)), (0, (6, 8), (6, 1)), (0, (6, 8), (1, 8)), (1, (4, 9), (4, 9)),
    (2, (5, 6), (5, 6)), (3, (3, 10), (3, 10)), (4, (7, 5), (7, 5)), (5, (6, 6), (6, 6)),
    (6, (4, 4), (4, 4)), (7, (3, 5), (3, 5)), (8, (5, 3), (5, 3)), (9, (4, 6), (6, 4)),
    (9, (3, 8), (8, 1)),
]


def main():
    if ref is None:
        sys.exit("oracle/_ref/libjasref.so not built (needs the reference checkout)")
    g = {}
    seed = 100
    for n, (eid, sa, sb) in enumerate(EXPR_CASES):
        a = normal(sa, seed, 2 * n)
        b = normal(sb, seed, 2 * n + 1)
        if eid in (2, 6):  # keep divisors away from 0
            b = (np.abs(b) + 0.5).astype(np.float32)
            a = (np.abs(a) + 0.5).astype(np.float32)
        r = np.zeros(1, np.int32)
        c = np.zeros(1, np.int32)
        ref.ref_expr(eid, fp(a), sa[0], sa[1], fp(b), sb[0], sb[1], None, ip(r), ip(c))
        out = np.zeros((r[0], c[0]), np.float32)
        ref.ref_expr(eid, fp(a), sa[0], sa[1], fp(b), sb[0], sb[1], fp(out), ip(r), ip(c))
        g[f"expr{n}_id"] = np.array(eid)
        g[f"expr{n}_a"], g[f"expr{n}_b"], g[f"expr{n}_out"] = a, b, out

    R, Cc = 9, 33
    x = normal((R, Cc), 1, 50)
    y = np.zeros_like(x)
    g["x"] = x
    ref.ref_hsoftmax(fp(x), R, Cc, fp(y)); g["hsoftmax"] = y.copy()
    ref.ref_softmax_global(fp(x), R, Cc, fp(y)); g["softmax_global"] = y.copy()
    ref.ref_layernorm_cols(fp(x), R, Cc, fp(y)); g["layernorm_cols"] = y.copy()
    ref.ref_relu(fp(x), R, Cc, fp(y)); g["relu"] = y.copy()
    ref.ref_sigmoid(fp(x), R, Cc, fp(y)); g["sigmoid"] = y.copy()
    hs, vs, hm, vmn, hmn = (np.zeros(k, np.float32) for k in (R, Cc, R, Cc, R))
    sc = np.zeros(3, np.float32)
    ref.ref_reductions(fp(x), R, Cc, fp(hs), fp(vs), fp(hm), fp(vmn), fp(hmn), fp(sc))
    g.update(hsum=hs, vsum=vs, hmax=hm, vmean=vmn, hmean=hmn, sum_max_mean=sc)

    a, b, c = normal((R, Cc), 1, 51), normal((R, Cc), 1, 52), normal((R, Cc), 1, 53)
    d = np.zeros_like(a)
    ref.ref_cfg2_expr(fp(a), fp(b), fp(c), fp(d), R, Cc)
    g.update(cfg2_a=a, cfg2_b=b, cfg2_c=c, cfg2_d=d)

    M, N, K = 11, 7, 13
    A, B = normal((M, K), 1, 54), normal((K, N), 1, 55)
    Cm = np.zeros((M, N), np.float32)
    ref.ref_gemm(M, N, K, fp(A), fp(B), fp(Cm))
    g.update(gemm_a=A, gemm_b=B, gemm_c=Cm)

    W, bb, X = normal((10, 12), 1, 56, std=0.3), normal(10, 1, 57), normal((12, 5), 1, 58)
    Y = np.zeros((10, 5), np.float32)
    ref.ref_linear(fp(W), fp(bb), fp(X), 10, 12, 5, fp(Y))
    g.update(linear_w=W, linear_b=bb, linear_x=X, linear_y=Y)

    dh, T, Tk = 8, 6, 5
    Wh = normal(3 * (dh * dh + dh), 1, 59, std=0.3)
    Xq, Xk = normal((dh, T), 1, 60), normal((dh, Tk), 1, 61)
    for mask in (0, 1):
        Yh = np.zeros((dh, T), np.float32)
        ref.ref_head(fp(Xq), None, dh, T, T, fp(Wh), mask, fp(Yh))
        g[f"head_self_m{mask}"] = Yh
    Yh = np.zeros((dh, T), np.float32)
    ref.ref_head(fp(Xq), fp(Xk), dh, T, Tk, fp(Wh), 0, fp(Yh))
    g.update(head_w=Wh, head_xq=Xq, head_xk=Xk, head_cross=Yh)

    d, H = 12, 3
    nm = 3 * H * ((d // H) ** 2 + d // H) + d * d + d
    Wm = normal(nm, 1, 62, std=0.3)
    Xm = normal((d, T), 1, 63)
    Ym = np.zeros((d, T), np.float32)
    ref.ref_mha(fp(Xm), None, d, H, T, T, fp(Wm), 1, fp(Ym))
    g.update(mha_w=Wm, mha_x=Xm, mha_y=Ym)

    Xr = normal((16, 6), 1, 64)
    Yr = np.zeros_like(Xr)
    ref.ref_rope(fp(Xr), 16, 6, fp(Yr))
    g.update(rope_x=Xr, rope_y=Yr)

    ne, nd, Te, Td = 2, 2, 4, 5
    nt = ref.ref_transformer_nparams(d, H, ne, nd)
    Wt = normal(nt, 1, 65, std=0.3)
    en, de = normal((d, Te), 1, 66), normal((d, Td), 1, 67)
    Yt = np.zeros((d, Td), np.float32)
    ref.ref_transformer(fp(en), Te, fp(de), Td, d, H, ne, nd, fp(Wt), fp(Yt))
    g.update(tf_w=Wt, tf_en=en, tf_de=de, tf_y=Yt, tf_dims=np.array([d, H, ne, nd, Te, Td]))
    # causal-prefix invariant of the reference decoder (transformer_test.hpp:246-282):
    # the first 3 output columns for the 3-token prefix
    Yp = np.zeros((d, 3), np.float32)
    ref.ref_transformer(fp(en), Te, fp(np.ascontiguousarray(de[:, :3])), 3, d, H, ne, nd, fp(Wt), fp(Yp))
    g["tf_prefix3"] = Yp

    # head dims the fused all-heads path takes (32, 64, 128): self attention with the mask, cross
    # attention, and an encoder-decoder stack with its causal-prefix invariant
    for tag, (d2, H2, T2, Tk2, seed) in {"mha32": (64, 2, 40, 23, 70), "mha64": (128, 2, 33, 19, 74),
                                                  "mha128": (128, 1, 29, 21, 90)}.items():
        n2 = 3 * H2 * ((d2 // H2) ** 2 + d2 // H2) + d2 * d2 + d2
        W2 = normal(n2, 1, seed, std=0.1)
        X2, K2 = normal((d2, T2), 1, seed + 1), normal((d2, Tk2), 1, seed + 2)
        Ys, Yc = np.zeros((d2, T2), np.float32), np.zeros((d2, T2), np.float32)
        ref.ref_mha(fp(X2), None, d2, H2, T2, T2, fp(W2), 1, fp(Ys))
        ref.ref_mha(fp(X2), fp(K2), d2, H2, T2, Tk2, fp(W2), 0, fp(Yc))
        g.update({f"{tag}_w": W2, f"{tag}_x": X2, f"{tag}_xk": K2, f"{tag}_self": Ys, f"{tag}_cross": Yc,
                  f"{tag}_dims": np.array([d2, H2, T2, Tk2])})
    d3, H3, ne3, nd3, Te3, Td3 = 64, 2, 1, 2, 20, 17
    W3 = normal(ref.ref_transformer_nparams(d3, H3, ne3, nd3), 1, 78, std=0.1)
    en3, de3 = normal((d3, Te3), 1, 79), normal((d3, Td3), 1, 80)
    Y3, Y3p = np.zeros((d3, Td3), np.float32), np.zeros((d3, 5), np.float32)
    ref.ref_transformer(fp(en3), Te3, fp(de3), Td3, d3, H3, ne3, nd3, fp(W3), fp(Y3))
    ref.ref_transformer(fp(en3), Te3, fp(np.ascontiguousarray(de3[:, :5])), 5, d3, H3, ne3, nd3, fp(W3), fp(Y3p))
    en3b, Y3b = normal((d3, Te3 + 3), 1, 81), np.zeros((d3, Td3), np.float32)  # a second, longer encoder input
    ref.ref_transformer(fp(en3b), Te3 + 3, fp(de3), Td3, d3, H3, ne3, nd3, fp(W3), fp(Y3b))
    g.update(tf32_en2=en3b, tf32_y2=Y3b)
    g.update(tf32_w=W3, tf32_en=en3, tf32_de=de3, tf32_y=Y3, tf32_prefix5=Y3p,
             tf32_dims=np.array([d3, H3, ne3, nd3, Te3, Td3]))

    # the prefix-recompute decode loop (transformer_test.hpp:227-239): per-head path (d_h 4)
    # and the fused path (d_h 32), 6 steps each
    for tag, (dp, Hp, nep, ndp, Tep, seed) in {"pred4": (12, 3, 2, 2, 5, 84), "pred32": (64, 2, 1, 2, 9, 88)}.items():
        Wp = normal(ref.ref_transformer_nparams(dp, Hp, nep, ndp), 1, seed, std=0.1)
        enp, dep = normal((dp, Tep), 1, seed + 1), normal(dp, 1, seed + 2)
        steps = 6
        Yp = np.zeros((dp, steps + 1), np.float32)
        ref.ref_predict_loop(fp(enp), Tep, fp(dep), dp, Hp, nep, ndp, fp(Wp), steps, fp(Yp))
        g.update({f"{tag}_w": Wp, f"{tag}_en": enp, f"{tag}_de0": dep, f"{tag}_y": Yp,
                  f"{tag}_dims": np.array([dp, Hp, nep, ndp, Tep, steps])})

    np.savez_compressed(OUT, **g)
    print("wrote", OUT, os.path.getsize(OUT), "bytes,", len(g), "arrays")


if __name__ == "__main__":
    main()
