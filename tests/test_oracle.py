"""Pin the CPU oracle (oracle/oracle.c) before trusting it as the GPU checker.

Pinning per function:
  * golden vectors written by the jasmine reference itself (tests/golden/jasmine_golden.npz,
    made by tests/golden/make_golden.py from oracle/_ref): gemm, linear, relu, sigmoid,
    hsoftmax, global softmax, column LayerNorm, all reductions, the config-2 expression,
    one jasmine head (masked/unmasked/cross), mat_mha_t, jasmine RoPE, and the full
    transformer_base_t encoder->decoder forward -- all BIT-EXACT;
  * live comparison against oracle/_ref on fresh random inputs when it is built;
  * closed forms / invariants / brute force for the ops jasmine lacks: tanh/GELU/SiLU vs
    libm double formulas, row LayerNorm (mean 0, var 1), RMSNorm (rms 1), softmax (rows sum
    to 1, shift invariance), LLaMA RoPE (norm preserving, relative-position dot products),
    attention vs a numpy fp64 brute force, argmax by brute force, the LM's KV-cache
    generation vs a cache-free recompute of every prefix, and LLaMA/GPT-2 blocks vs a numpy
    transcription of the textbook formulas.
"""
import math
import os

import numpy as np
import pytest

from oracle_lib import orc, ref, fp, ip, normal, randint, LmCfg, LmWeights, LM_WEIGHT_FIELDS

GOLD = os.path.join(os.path.dirname(__file__), "golden", "jasmine_golden.npz")
pytestmark = pytest.mark.skipif(orc is None, reason="oracle/liboracle.so not built")


@pytest.fixture(scope="module")
def g():
    return np.load(GOLD)


def bits_equal(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_golden_gemm_linear(g):
    A, B = g["gemm_a"], g["gemm_b"]
    M, K = A.shape
    N = B.shape[1]
    C = np.zeros((M, N), np.float32)
    orc.orc_gemm(M, N, K, fp(A), K, 1, fp(B), N, 1, fp(C), N)
    assert bits_equal(C, g["gemm_c"])
    W, b, X = g["linear_w"], g["linear_b"], g["linear_x"]
    Y = np.zeros_like(g["linear_y"])
    orc.orc_linear(fp(W), fp(b), fp(X), W.shape[0], W.shape[1], X.shape[1], fp(Y))
    assert bits_equal(Y, g["linear_y"])


def test_golden_rowops(g):
    x = g["x"]
    R, Cc = x.shape
    y = np.zeros_like(x)
    for name, fn in (("hsoftmax", orc.orc_hsoftmax), ("softmax_global", orc.orc_softmax_global)):
        fn(fp(x), R, Cc, fp(y))
        assert bits_equal(y, g[name]), name
    orc.orc_layernorm_cols_jas(fp(x), R, Cc, None, None, fp(y))
    assert bits_equal(y, g["layernorm_cols"])
    orc.orc_relu(fp(x), x.size, fp(y))
    assert bits_equal(y, g["relu"])
    orc.orc_sigmoid(fp(x), x.size, fp(y))
    assert bits_equal(y, g["sigmoid"])


def test_golden_reductions(g):
    x = g["x"]
    R, Cc = x.shape
    for name, fn, n in (("hsum", orc.orc_hsum, R), ("vsum", orc.orc_vsum, Cc), ("hmax", orc.orc_hmax, R),
                        ("vmean", orc.orc_vmean, Cc), ("hmean", orc.orc_hmean, R)):
        o = np.zeros(n, np.float32)
        fn(fp(x), R, Cc, fp(o))
        assert bits_equal(o, g[name]), name
    s = g["sum_max_mean"]
    assert np.float32(orc.orc_sum(fp(x), R, Cc)) == s[0]
    assert np.float32(orc.orc_max(fp(x), R, Cc)) == s[1]
    assert np.float32(np.float32(orc.orc_sum(fp(x), R, Cc)) / np.float32(R * Cc)) == s[2]


def test_golden_cfg2_expr(g):
    a, b, c = g["cfg2_a"], g["cfg2_b"], g["cfg2_c"]
    d = np.zeros_like(a)
    orc.orc_cfg2_expr(fp(a), fp(b), fp(c), fp(d), a.size)
    assert bits_equal(d, g["cfg2_d"])


def _head_args(W, dh):
    o = [0, dh * dh, dh * dh + dh, 2 * dh * dh + dh, 2 * dh * dh + 2 * dh, 3 * dh * dh + 2 * dh]
    return [fp(W[k:]) for k in o]


def test_golden_attention(g):
    W, Xq, Xk = g["head_w"], g["head_xq"], g["head_xk"]
    dh, T = Xq.shape
    Tk = Xk.shape[1]
    for mask in (0, 1):
        Y = np.zeros((dh, T), np.float32)
        orc.orc_jas_head(fp(Xq), fp(Xq), dh, T, T, *_head_args(W, dh), mask, fp(Y))
        assert bits_equal(Y, g[f"head_self_m{mask}"]), mask
    Y = np.zeros((dh, T), np.float32)
    orc.orc_jas_head(fp(Xq), fp(Xk), dh, T, Tk, *_head_args(W, dh), 0, fp(Y))
    assert bits_equal(Y, g["head_cross"])
    Wm, Xm = g["mha_w"], g["mha_x"]
    d, T = Xm.shape
    Y = np.zeros((d, T), np.float32)
    orc.orc_jas_mha(fp(Xm), fp(Xm), d, 3, T, T, fp(Wm), 1, fp(Y))
    assert bits_equal(Y, g["mha_y"])
    # the fused-heads fixtures (head dims 32, 64, 128): masked self and cross attention
    for tag in ("mha32", "mha64", "mha128"):
        d2, H2, T2, Tk2 = (int(v) for v in g[f"{tag}_dims"])
        W2, X2, K2 = g[f"{tag}_w"], g[f"{tag}_x"], g[f"{tag}_xk"]
        Ys, Yc = np.zeros((d2, T2), np.float32), np.zeros((d2, T2), np.float32)
        orc.orc_jas_mha(fp(X2), fp(X2), d2, H2, T2, T2, fp(W2), 1, fp(Ys))
        orc.orc_jas_mha(fp(X2), fp(K2), d2, H2, T2, Tk2, fp(W2), 0, fp(Yc))
        assert bits_equal(Ys, g[f"{tag}_self"]), tag
        assert bits_equal(Yc, g[f"{tag}_cross"]), tag


def test_golden_rope_and_transformer(g):
    X = g["rope_x"]
    Y = np.zeros_like(X)
    orc.orc_rope_jas(fp(X), X.shape[0], X.shape[1], fp(Y))
    assert bits_equal(Y, g["rope_y"])
    d, H, ne, nd, Te, Td = [int(v) for v in g["tf_dims"]]
    Yt = np.zeros((d, Td), np.float32)
    orc.orc_jas_transformer(fp(g["tf_en"]), Te, fp(g["tf_de"]), Td, d, H, ne, nd, fp(g["tf_w"]), fp(Yt))
    assert bits_equal(Yt, g["tf_y"])
    # the reference's causal-prefix invariant holds exactly for the golden decoder
    assert bits_equal(np.ascontiguousarray(g["tf_y"][:, :3]), g["tf_prefix3"])


def test_rope_jasmine_known_answer():
    # mat_RoPE_t.hpp:113 closed form: block (i, m) = [cos(2m t), -sin((2m+1) t); sin(2m t), cos((2m+1) t)]
    # with t = 10000^-(i/d).  d = 4, i = 1, m = 1 -> t = 0.1 -> [cos .2, -sin .3; sin .2, cos .3]
    d, T = 4, 2
    X = np.zeros((d, T), np.float32)
    X[2, 1] = 1.0  # picks column 0 of block (i=1, m=1)
    Y = np.zeros_like(X)
    orc.orc_rope_jas(fp(X), d, T, fp(Y))
    assert abs(Y[2, 1] - math.cos(0.2)) < 1e-6 and abs(Y[3, 1] - math.sin(0.2)) < 1e-6
    X[:] = 0
    X[3, 1] = 1.0
    orc.orc_rope_jas(fp(X), d, T, fp(Y))
    assert abs(Y[2, 1] + math.sin(0.3)) < 1e-6 and abs(Y[3, 1] - math.cos(0.3)) < 1e-6


@pytest.mark.skipif(ref is None, reason="reference build (oracle/_ref) not present")
def test_live_against_reference():
    rng = np.random.default_rng(7)
    for R, Cc in ((3, 17), (12, 5), (31, 64)):
        x = rng.standard_normal((R, Cc)).astype(np.float32)
        y1, y2 = np.zeros_like(x), np.zeros_like(x)
        orc.orc_hsoftmax(fp(x), R, Cc, fp(y1)); ref.ref_hsoftmax(fp(x), R, Cc, fp(y2))
        assert bits_equal(y1, y2)
        orc.orc_layernorm_cols_jas(fp(x), R, Cc, None, None, fp(y1)); ref.ref_layernorm_cols(fp(x), R, Cc, fp(y2))
        assert bits_equal(y1, y2)
        b, c = rng.standard_normal((2, R, Cc)).astype(np.float32)
        orc.orc_cfg2_expr(fp(x), fp(b), fp(c), fp(y1), x.size); ref.ref_cfg2_expr(fp(x), fp(b), fp(c), fp(y2), R, Cc)
        assert bits_equal(y1, y2)
    d, H, T = 16, 4, 7
    W = (rng.standard_normal(orc.orc_jas_mha_nparams(d, H)) * 0.3).astype(np.float32)
    X = rng.standard_normal((d, T)).astype(np.float32)
    y1, y2 = np.zeros((d, T), np.float32), np.zeros((d, T), np.float32)
    orc.orc_jas_mha(fp(X), fp(X), d, H, T, T, fp(W), 1, fp(y1)); ref.ref_mha(fp(X), None, d, H, T, T, fp(W), 1, fp(y2))
    assert bits_equal(y1, y2)


def test_new_activation_closed_forms():
    for x in (-5.0, -1.3, -0.2, 0.0, 0.7, 2.5, 9.0):
        xf = float(np.float32(x))
        gelu = 0.5 * xf * (1 + math.tanh(math.sqrt(2 / math.pi) * (xf + 0.044715 * xf ** 3)))
        assert orc.orc_gelu(xf) == np.float32(gelu)
        assert orc.orc_silu(xf) == np.float32(xf / (1 + math.exp(-xf)))
    # GELU(x) ~ x for large x, ~0 for very negative x (tanh form limits)
    assert abs(orc.orc_gelu(8.0) - 8.0) < 1e-6 and abs(orc.orc_gelu(-8.0)) < 1e-6


def test_row_norms_invariants():
    x = normal((6, 257), 3, 1, mean=0.5, std=2.0)
    y = np.zeros_like(x)
    orc.orc_layernorm_rows(fp(x), 6, 257, 1e-5, None, None, fp(y))
    assert np.allclose(y.mean(1), 0, atol=1e-5) and np.allclose(y.var(1), 1, atol=1e-3)
    orc.orc_rmsnorm_rows(fp(x), 6, 257, 1e-6, None, fp(y))
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(1)), 1, atol=1e-5)
    # gains scale the output elementwise
    gvec = np.linspace(0.5, 2, 257).astype(np.float32)
    y2 = np.zeros_like(x)
    orc.orc_rmsnorm_rows(fp(x), 6, 257, 1e-6, fp(gvec), fp(y2))
    assert np.allclose(y2, y * gvec, rtol=1e-6)


def test_softmax_invariants():
    x = normal((5, 40), 4, 1, std=3.0)
    y, y2 = np.zeros_like(x), np.zeros_like(x)
    orc.orc_hsoftmax(fp(x), 5, 40, fp(y))
    assert np.allclose(y.sum(1), 1, atol=1e-6)
    xs = (x + np.float32(7.0)).astype(np.float32)
    orc.orc_hsoftmax(fp(xs), 5, 40, fp(y2))
    assert np.allclose(y, y2, atol=1e-6)


def test_llama_rope_properties():
    dh = 128
    q, k = normal(dh, 5, 1), normal(dh, 5, 2)
    dots = []
    for m, n in ((3, 1), (10, 8), (2000, 1998)):
        qm, kn = q.copy(), k.copy()
        orc.orc_rope_llama(fp(qm), dh, m, 10000.0)
        orc.orc_rope_llama(fp(kn), dh, n, 10000.0)
        assert abs(np.linalg.norm(qm) - np.linalg.norm(q)) < 1e-4  # rotation keeps the norm
        dots.append(float(np.dot(qm.astype(np.float64), kn)))
    assert max(dots) - min(dots) < 1e-3  # <R_m q, R_n k> depends only on m - n
    # pair 0 rotates by exactly pos radians (theta^0 = 1)
    v = np.zeros(dh, np.float32)
    v[0] = 1
    orc.orc_rope_llama(fp(v), dh, 1, 10000.0)
    assert abs(v[0] - math.cos(1)) < 1e-7 and abs(v[1] - math.sin(1)) < 1e-7


def _attn_numpy(Q, K, V, scale, causal):
    B, H, Sq, D = Q.shape
    Sk = K.shape[2]
    s = np.einsum("bhqd,bhkd->bhqk", Q.astype(np.float64), K.astype(np.float64)) * scale
    if causal:
        mask = np.arange(Sk)[None, :] > (np.arange(Sq)[:, None] + Sk - Sq)
        s[..., mask] = -np.inf
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", p, V.astype(np.float64))


@pytest.mark.parametrize("Sq,Sk,causal", [(9, 9, 1), (4, 11, 1), (6, 13, 0)])
def test_attention_brute_force(Sq, Sk, causal):
    B, H, D = 2, 3, 16
    Q, K, V = normal((B, H, Sq, D), 6, 1), normal((B, H, Sk, D), 6, 2), normal((B, H, Sk, D), 6, 3)
    O = np.zeros((B, H, Sq, D), np.float32)
    orc.orc_attention(fp(Q), fp(K), fp(V), fp(O), B, H, Sq, Sk, D, 1 / math.sqrt(D), causal)
    assert np.allclose(O, _attn_numpy(Q, K, V, 1 / math.sqrt(D), causal), atol=1e-6)


def test_argmax_brute():
    x = normal(1000, 8, 1)
    assert orc.orc_argmax(fp(x), 1000) == int(np.argmax(x))
    x[10] = x[500] = 100.0  # ties: first maximum
    assert orc.orc_argmax(fp(x), 1000) == 10


def test_rng_reproducible():
    a, b = normal(10, 1, 2), normal(10, 1, 2)
    assert bits_equal(a, b)
    big = normal(200000, 3, 0, std=0.02)
    assert abs(big.mean()) < 3e-4 and abs(big.std() - 0.02) < 3e-4
    ids = randint(10000, 256, 0)
    assert ids.min() >= 0 and ids.max() < 256 and len(np.unique(ids)) == 256


# ---------------------------------------------------------------- decoder LMs
def make_lm(kind, L=2, d=64, H=2, F=128, V=97, ctx=24, seed=11):
    cfg = LmCfg(kind, L, d, H, F, V, ctx, 1e-5 if kind == 0 else 1e-6, 10000.0)
    rs = np.random.default_rng(seed)
    w = {}

    def n(*s):
        return (rs.standard_normal(s) * 0.05).astype(np.float32)

    w["wte"] = n(V, d)
    w["ln1_g"] = (1 + n(L, d)).astype(np.float32)
    w["w_qkv"] = n(L, 3 * d, d)
    w["w_o"] = n(L, d, d)
    w["ln2_g"] = (1 + n(L, d)).astype(np.float32)
    w["lnf_g"] = (1 + n(d)).astype(np.float32)
    if kind == 0:
        w.update(wpe=n(ctx, d), ln1_b=n(L, d), b_qkv=n(L, 3 * d), b_o=n(L, d), ln2_b=n(L, d), w_fc=n(L, F, d),
                 b_fc=n(L, F), w_proj=n(L, d, F), b_proj=n(L, d), lnf_b=n(d))
    else:
        w.update(w_gate=n(L, F, d), w_up=n(L, F, d), w_down=n(L, d, F), w_head=n(V, d))
    lw = LmWeights(*[fp(w[f]) if f in w else None for f in LM_WEIGHT_FIELDS])
    return cfg, w, lw


def _bf16(a):
    """round to bf16 (nearest even) and back, elementwise, in fp64"""
    f = np.asarray(a, np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def _np_lm_logits(kind, cfg, w, ids, kv_round_from=None):
    """Cache-free numpy (fp64) forward of one sequence, logits of the last position.
    kv_round_from = P: query positions >= P see every key/value rounded to bf16 (a bf16 KV
    cache after a P-token prefill); positions < P see them unrounded."""
    L, d, H = cfg.n_layer, cfg.d_model, cfg.n_head
    dh = d // H
    T = len(ids)
    x = w["wte"][ids].astype(np.float64)
    if kind == 0:
        x = x + w["wpe"][:T]

    def norm(v, gk, bk, l):
        gg = w[gk][l] if l is not None else w[gk]
        if kind == 0:
            bb = w[bk][l] if l is not None else w[bk]
            mu = v.mean(-1, keepdims=True)
            return (v - mu) / np.sqrt(((v - mu) ** 2).mean(-1, keepdims=True) + cfg.eps) * gg + bb
        return v / np.sqrt((v ** 2).mean(-1, keepdims=True) + cfg.eps) * gg

    def rope(v):  # v [T, H, dh]
        i = np.arange(dh // 2)
        ang = np.arange(T)[:, None] * (cfg.rope_theta ** (-2.0 * i / dh))[None, :]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        x0, x1 = v[..., 0::2], v[..., 1::2]
        out = np.empty_like(v)
        out[..., 0::2] = x0 * c - x1 * s
        out[..., 1::2] = x0 * s + x1 * c
        return out

    for l in range(L):
        h = norm(x, "ln1_g", "ln1_b", l)
        qkv = h @ w["w_qkv"][l].T + (w["b_qkv"][l] if kind == 0 else 0)
        q, k, v = (qkv[:, i * d:(i + 1) * d].reshape(T, H, dh) for i in range(3))
        if kind == 1:
            q, k = rope(q), rope(k)
        def attend(kk, vv):
            s = np.einsum("thd,uhd->htu", q, kk) / math.sqrt(dh)
            s[:, np.triu(np.ones((T, T), bool), 1)] = -np.inf
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            return np.einsum("htu,uhd->thd", p, vv).reshape(T, d)
        a = attend(k, v)
        if kv_round_from is not None and T > kv_round_from:
            a[kv_round_from:] = attend(_bf16(k), _bf16(v))[kv_round_from:]
        x = x + a @ w["w_o"][l].T + (w["b_o"][l] if kind == 0 else 0)
        h = norm(x, "ln2_g", "ln2_b", l)
        if kind == 0:
            u = h @ w["w_fc"][l].T + w["b_fc"][l]
            u = 0.5 * u * (1 + np.tanh(math.sqrt(2 / math.pi) * (u + 0.044715 * u ** 3)))
            x = x + u @ w["w_proj"][l].T + w["b_proj"][l]
        else:
            gt, up = h @ w["w_gate"][l].T, h @ w["w_up"][l].T
            x = x + (gt / (1 + np.exp(-gt)) * up) @ w["w_down"][l].T
    hf = norm(x[-1:], "lnf_g", "lnf_b", None)
    head = w["wte"] if kind == 0 else w["w_head"]
    return (hf @ head.T)[0]


@pytest.mark.parametrize("kind", [0, 1])
def test_lm_oracle_bf16_kv_cache(kind):
    """kv_bf16: the oracle's cache rounding equals the parallel numpy form (queries from the
    prompt see unrounded keys/values, generated ones see them all rounded); the first step
    (the prompt's last token) is unchanged, later steps move by about the bf16 rounding."""
    cfg, w, lw = make_lm(kind)
    cfg_r, _, _ = make_lm(kind)
    cfg_r.kv_bf16 = 1
    B, P, steps = 2, 5, 5
    prompt = randint((B, P), cfg.vocab, 3)
    ids, ids_r = np.zeros((B, steps), np.int32), np.zeros((B, steps), np.int32)
    lg, lg_r = np.zeros((steps, B, cfg.vocab), np.float32), np.zeros((steps, B, cfg.vocab), np.float32)
    orc.orc_lm_generate(cfg, lw, B, P, ip(prompt), steps, None, ip(ids), fp(lg), 1)
    force = np.ascontiguousarray(ids)  # same token stream for both
    orc.orc_lm_generate(cfg_r, lw, B, P, ip(prompt), steps, ip(force), ip(ids_r), fp(lg_r), 1)
    assert np.array_equal(lg[0], lg_r[0])
    assert not np.array_equal(lg[1:], lg_r[1:])
    assert np.abs(lg - lg_r).max() < 5e-3
    for b in range(B):
        seq = list(prompt[b])
        for s in range(steps):
            ref_l = _np_lm_logits(kind, cfg, w, np.array(seq), kv_round_from=P)
            assert np.allclose(lg_r[s, b], ref_l, atol=1e-4), (b, s)
            seq.append(int(force[b, s]))


@pytest.mark.parametrize("kind", [0, 1])
def test_lm_oracle_vs_numpy_and_kv_invariant(kind):
    cfg, w, lw = make_lm(kind)
    B, P, steps = 2, 5, 6
    prompt = randint((B, P), cfg.vocab, 1)
    ids = np.zeros((B, steps), np.int32)
    logits = np.zeros((steps, B, cfg.vocab), np.float32)
    orc.orc_lm_generate(cfg, lw, B, P, ip(prompt), steps, None, ip(ids), fp(logits), 2)
    for b in range(B):
        seq = list(prompt[b])
        for s in range(steps):
            ref_l = _np_lm_logits(kind, cfg, w, np.array(seq))
            assert np.allclose(logits[s, b], ref_l, atol=1e-4), (b, s)
            assert ids[b, s] == int(np.argmax(logits[s, b]))
            seq.append(int(ids[b, s]))
        # KV-cache generation == cache-free recompute of the whole prefix (last column)
        full = np.array(seq[:-1], np.int32)[None, :]
        last = np.zeros((1, cfg.vocab), np.float32)
        orc.orc_lm_last_logits(cfg, lw, 1, full.shape[1], ip(full), fp(last), 1)
        assert np.allclose(last[0], logits[-1, b], atol=1e-6)
