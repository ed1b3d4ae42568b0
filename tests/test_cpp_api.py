"""The C++20 jasmine-compatible API (jasmine_amd/include) against the reference's outputs.

tests/cpp/api_driver.cpp is written as jasmine user code (mat_t, views, expressions, nets,
mat_mha_t, transformer_base_t, weights through an init_t<> hook) and compiled against this
project's headers into tests/cpp/libjasapi.so.  Each api_X entry point gets the inputs the
reference's ref_X call got when tests/golden/jasmine_golden.npz was written, so these tests
compare the device path of the C++ API with the reference's own outputs.

Tolerance (fp32): |api - ref| <= 1e-3 + 1e-4 |ref|; elementwise +-*/ trees and per-row /
per-column reductions are also checked bit-exact, as their arithmetic order is jasmine's.
"""
import ctypes
import math
import os

import numpy as np
import pytest

from oracle_lib import fp, ip

HERE = os.path.dirname(os.path.abspath(__file__))
# JAS_API_SO selects another build of the driver (the sanitizer build, libjasapi_san.so)
LIB = os.environ.get("JAS_API_SO") or os.path.join(HERE, "cpp", "libjasapi.so")
GOLD = os.path.join(HERE, "golden", "jasmine_golden.npz")


def load_api():
    if not os.path.exists(LIB):
        raise RuntimeError(f"{LIB} is not built (make -C tests/cpp, or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB)
    lib.api_last_error.restype = ctypes.c_char_p
    lib.api_transformer_nparams.restype = ctypes.c_long
    return lib


@pytest.fixture(scope="module")
def api():
    return load_api()


@pytest.fixture(scope="module")
def g():
    return np.load(GOLD)


def ok(lib, rc):
    assert rc == 0, lib.api_last_error().decode()


def close(a, b, atol=1e-3, rtol=1e-4):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    assert np.all(np.isfinite(a) == np.isfinite(b)), "non-finite mismatch"
    fin = np.isfinite(b)
    err = np.abs(a - b)[fin]
    assert np.all(err <= atol + rtol * np.abs(b)[fin]), f"max abs err {err.max():.3g}"


def bitexact(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


# ------------------------------------------------------------------ CPU (no device calls)
def test_api_library_exports(api):
    for name in ("api_gemm", "api_gemm_tn", "api_cfg2_expr", "api_expr", "api_hsoftmax", "api_softmax_global",
                 "api_reductions", "api_linear", "api_relu", "api_sigmoid", "api_layernorm_cols", "api_head",
                 "api_mha", "api_rope", "api_transformer", "api_transformer_nparams", "api_last_error", "api_set_fused_heads", "api_transformer_reencode", "api_predict_loop",
                 "api_expr_deferred", "api_bf16_expr", "api_bf16_gemm", "api_bf16_hsoftmax", "api_bf16_reductions",
                 "api_bf16_linear"):
        assert hasattr(api, name), name


@pytest.mark.parametrize("d,H,ne,nd", [(12, 3, 2, 2), (8, 2, 1, 3), (16, 4, 3, 1)])
def test_api_transformer_parameter_walk(api, d, H, ne, nd):
    """init_weight visits what the reference visits: per head Wq,bq,Wk,bk,Wv,bv (dh x dh + dh)
    and the output projection (d x d + d) per attention block, then the FFN weight (d x d + d);
    the encoder layer has one attention block, the decoder layer two.  layer_norm_net_t
    creates gamma/beta at its first forward (mat_net_t.hpp:209-224), so no LN parameter is
    visited."""
    dh = d // H
    mha = 3 * H * (dh * dh + dh) + d * d + d
    ffn = d * d + d
    want = ne * (mha + ffn) + nd * (2 * mha + ffn)
    assert api.api_transformer_nparams(d, H, ne, nd) == want
    if "_ref" in os.listdir(os.path.join(os.path.dirname(HERE), "oracle")):
        from oracle_lib import ref
        if ref is not None:
            assert ref.ref_transformer_nparams(d, H, ne, nd) == want


# ------------------------------------------------------------------ GPU parity
@pytest.mark.gpu
def test_api_expressions(api, g):
    n = 0
    while f"expr{n}_id" in g:
        eid = int(g[f"expr{n}_id"])
        a, b, want = g[f"expr{n}_a"], g[f"expr{n}_b"], g[f"expr{n}_out"]
        r, c = np.zeros(1, np.int32), np.zeros(1, np.int32)
        out = np.zeros(want.shape, np.float32)
        ok(api, api.api_expr(eid, fp(a), a.shape[0], a.shape[1], fp(b), b.shape[0], b.shape[1], fp(out), ip(r), ip(c)))
        assert (r[0], c[0]) == want.shape
        close(out, want)
        if eid not in (3, 4):  # exp / sigmoid go through libm-class functions
            assert bitexact(out, want), (n, eid)
        n += 1
    assert n >= 13


@pytest.mark.gpu
def test_api_cfg2_expression(api, g):
    a, b, c, want = g["cfg2_a"], g["cfg2_b"], g["cfg2_c"], g["cfg2_d"]
    d = np.zeros_like(a)
    ok(api, api.api_cfg2_expr(fp(a), fp(b), fp(c), fp(d), a.shape[0], a.shape[1]))
    close(d, want)


@pytest.mark.gpu
def test_api_expression_kept_in_a_variable(api):
    """`auto e = a * b + a * 0.5f - (b + 1.0f) * 2.0f;` evaluated statements later (after other
    temporaries reused the stack): the nodes hold their sub-expressions by value."""
    rng = np.random.default_rng(5)
    a = rng.standard_normal((37, 29)).astype(np.float32)
    b = rng.standard_normal((37, 29)).astype(np.float32)
    out = np.zeros_like(a)
    ok(api, api.api_expr_deferred(fp(a), fp(b), fp(out), 37, 29))
    f = np.float32
    want = (a * b + a * f(0.5)) - (b + f(1.0)) * f(2.0)
    assert bitexact(out, want)


@pytest.mark.gpu
def test_api_row_and_column_ops(api, g):
    x = g["x"]
    R, C = x.shape
    for fn, key in ((api.api_hsoftmax, "hsoftmax"), (api.api_softmax_global, "softmax_global"),
                    (api.api_layernorm_cols, "layernorm_cols"), (api.api_relu, "relu"),
                    (api.api_sigmoid, "sigmoid")):
        y = np.zeros_like(x)
        ok(api, fn(fp(x), R, C, fp(y)))
        close(y, g[key], atol=1e-5, rtol=1e-5)
    y = np.zeros_like(x)
    ok(api, api.api_relu(fp(x), R, C, fp(y)))
    assert bitexact(y, g["relu"])


@pytest.mark.gpu
def test_api_reductions(api, g):
    x = g["x"]
    R, C = x.shape
    hs, vs, hm, vmn, hmn = (np.zeros(k, np.float32) for k in (R, C, R, C, R))
    sc = np.zeros(3, np.float32)
    ok(api, api.api_reductions(fp(x), R, C, fp(hs), fp(vs), fp(hm), fp(vmn), fp(hmn), fp(sc)))
    for got, key in ((hs, "hsum"), (vs, "vsum"), (hm, "hmax"), (vmn, "vmean"), (hmn, "hmean")):
        assert bitexact(got, g[key].reshape(got.shape)), key
    close(sc, g["sum_max_mean"], atol=1e-5, rtol=1e-5)


@pytest.mark.gpu
def test_api_gemm_and_linear(api, g):
    A, B, want = g["gemm_a"], g["gemm_b"], g["gemm_c"]
    M, K = A.shape
    N = B.shape[1]
    C = np.zeros((M, N), np.float32)
    ok(api, api.api_gemm(M, N, K, fp(A), fp(B), fp(C)))
    close(C, want, atol=1e-5, rtol=1e-5)
    At = np.ascontiguousarray(A.T)
    ok(api, api.api_gemm_tn(M, N, K, fp(At), fp(B), fp(C)))
    close(C, want, atol=1e-5, rtol=1e-5)
    W, b, X, want = g["linear_w"], g["linear_b"], g["linear_x"], g["linear_y"]
    Y = np.zeros_like(want)
    ok(api, api.api_linear(fp(W), fp(b), fp(X), W.shape[0], W.shape[1], X.shape[1], fp(Y)))
    close(Y, want, atol=1e-5, rtol=1e-5)


@pytest.mark.gpu
def test_api_head(api, g):
    Wh, Xq, Xk = g["head_w"], g["head_xq"], g["head_xk"]
    dh, T = Xq.shape
    Tk = Xk.shape[1]
    for mask in (0, 1):
        Y = np.zeros((dh, T), np.float32)
        ok(api, api.api_head(fp(Xq), None, dh, T, T, fp(Wh), mask, fp(Y)))
        close(Y, g[f"head_self_m{mask}"])
    Y = np.zeros((dh, T), np.float32)
    ok(api, api.api_head(fp(Xq), fp(Xk), dh, T, Tk, fp(Wh), 0, fp(Y)))
    close(Y, g["head_cross"])


@pytest.mark.gpu
def test_api_mha(api, g):
    Wm, Xm, want = g["mha_w"], g["mha_x"], g["mha_y"]
    d, T = Xm.shape
    Y = np.zeros_like(want)
    ok(api, api.api_mha(fp(Xm), None, d, 3, T, T, fp(Wm), 1, fp(Y)))
    close(Y, want)


@pytest.mark.gpu
def test_api_rope(api, g):
    X, want = g["rope_x"], g["rope_y"]
    Y = np.zeros_like(X)
    ok(api, api.api_rope(fp(X), X.shape[0], X.shape[1], fp(Y)))
    close(Y, want, atol=1e-6, rtol=1e-5)


@pytest.mark.gpu
def test_api_transformer(api, g):
    d, H, ne, nd, Te, Td = (int(v) for v in g["tf_dims"])
    Wt, en, de = g["tf_w"], g["tf_en"], g["tf_de"]
    Y = np.zeros((d, Td), np.float32)
    ok(api, api.api_transformer(fp(en), Te, fp(de), Td, d, H, ne, nd, fp(Wt), fp(Y)))
    close(Y, g["tf_y"])
    # causal prefix: the first 3 decoder columns alone give the reference's 3-token output
    Yp = np.zeros((d, 3), np.float32)
    ok(api, api.api_transformer(fp(en), Te, fp(np.ascontiguousarray(de[:, :3])), 3, d, H, ne, nd, fp(Wt), fp(Yp)))
    close(Yp, g["tf_prefix3"])
    close(Y[:, :3], Yp)


def _mha_case(api, g, tag, cross):
    d, H, T, Tk = (int(v) for v in g[f"{tag}_dims"])
    Y = np.zeros((d, T), np.float32)
    if cross:
        ok(api, api.api_mha(fp(g[f"{tag}_x"]), fp(g[f"{tag}_xk"]), d, H, T, Tk, fp(g[f"{tag}_w"]), 0, fp(Y)))
    else:
        ok(api, api.api_mha(fp(g[f"{tag}_x"]), None, d, H, T, T, fp(g[f"{tag}_w"]), 1, fp(Y)))
    return Y


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["mha32", "mha64", "mha128"])
@pytest.mark.parametrize("cross", [0, 1])
def test_api_mha_fused_heads(api, g, tag, cross):
    """Head dims 32 / 64 / 128: every head in batched projections plus the flash kernel, against
    the reference's outputs; the per-head path (materialised scores) agrees with both."""
    Y = _mha_case(api, g, tag, cross)
    close(Y, g[f"{tag}_cross" if cross else f"{tag}_self"])
    api.api_set_fused_heads(0)
    try:
        Yp = _mha_case(api, g, tag, cross)
    finally:
        api.api_set_fused_heads(1)
    close(Yp, g[f"{tag}_cross" if cross else f"{tag}_self"])
    close(Y, Yp, atol=1e-4, rtol=1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [1, 0])
def test_api_transformer_head_dim_32(api, g, fused):
    d, H, ne, nd, Te, Td = (int(v) for v in g["tf32_dims"])
    api.api_set_fused_heads(fused)
    try:
        Y = np.zeros((d, Td), np.float32)
        ok(api, api.api_transformer(fp(g["tf32_en"]), Te, fp(g["tf32_de"]), Td, d, H, ne, nd, fp(g["tf32_w"]), fp(Y)))
        close(Y, g["tf32_y"])
        Yp = np.zeros((d, 5), np.float32)
        de5 = np.ascontiguousarray(g["tf32_de"][:, :5])
        ok(api, api.api_transformer(fp(g["tf32_en"]), Te, fp(de5), 5, d, H, ne, nd, fp(g["tf32_w"]), fp(Yp)))
        close(Yp, g["tf32_prefix5"])
        close(Y[:, :5], Yp)
    finally:
        api.api_set_fused_heads(1)


@pytest.mark.gpu
def test_api_transformer_reencode(api, g):
    """The decoder's cross attention keeps the encoder-side keys / values between forwards;
    a new encoder_forward must replace them (its output is a new matrix state)."""
    d, H, ne, nd, Te, Td = (int(v) for v in g["tf32_dims"])
    en2 = g["tf32_en2"]
    Y1, Y2, Y3 = (np.zeros((d, Td), np.float32) for _ in range(3))
    ok(api, api.api_transformer_reencode(fp(g["tf32_en"]), Te, fp(en2), en2.shape[1], fp(g["tf32_de"]), Td, d, H, ne,
                                         nd, fp(g["tf32_w"]), fp(Y1), fp(Y2), fp(Y3)))
    close(Y1, g["tf32_y"])
    close(Y2, g["tf32_y2"])
    assert np.array_equal(Y2, Y3)


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["pred4", "pred32"])
def test_api_predict_loop(api, g, tag):
    """The reference's autoregressive loop (test_transformer_t::predict without its flag
    rows): decoder forward on a growing prefix view, last output column appended, 6 steps.
    d_h 4 runs the per-head path, d_h 32 the fused one."""
    d, H, ne, nd, Te, steps = (int(v) for v in g[f"{tag}_dims"])
    Y = np.zeros((d, steps + 1), np.float32)
    ok(api, api.api_predict_loop(fp(g[f"{tag}_en"]), Te, fp(g[f"{tag}_de0"]), d, H, ne, nd, fp(g[f"{tag}_w"]), steps,
                                 fp(Y)))
    close(Y, g[f"{tag}_y"])


# ------------------------------------------------------------------ mat_t<jas::bf16>
# The same user code with bf16 matrices.  Two checks per operation:
#  * against a numpy model of bf16 arithmetic (float32 operation, then round to nearest even,
#    per node, with the promotion rule: bf16 with bf16 or an integer stays bf16, with float or
#    double widens) -- bit-exact where only + - * / and comparisons are involved, within one
#    bf16 ulp where a libm-class function or an fp32 accumulation sits before the rounding;
#  * against the reference's own fp32 outputs (golden) at the bf16 tolerance 5e-2 + 2e-2 |ref|.
BF_ATOL, BF_RTOL = 5e-2, 2e-2


def rb(x):
    """float32 -> bf16 -> float32, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def bcast(x, R, C):  # jasmine's modulo broadcast (mat_t.hpp:304-305)
    return x[np.arange(R)[:, None] % x.shape[0], np.arange(C)[None, :] % x.shape[1]]


def within_ulp(got, want):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    return np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)


def bf16_model(eid, a, b, R, C):
    f32, f64 = np.float32, np.float64
    if eid == 9:
        A, B = bcast(rb(a).T, R, C), bcast(rb(b), R, C)
        return A.astype(f64) * 0.25 + B.astype(f64)
    A, B = bcast(rb(a), R, C), bcast(rb(b), R, C)
    with np.errstate(all="ignore"):
        if eid == 0: return rb(A + B)
        if eid == 1: return rb(A - rb(B * f32(2)))
        if eid == 2: return rb(A * B).astype(f64) / (B.astype(f64) + 3.0)
        if eid == 3: return rb(np.exp(rb(A - B)))
        if eid == 4: return rb((1.0 / (1.0 + np.exp(-rb(A * B)).astype(f64))).astype(f32))
        if eid == 5: return rb(rb((A > B).astype(f32) * A) + rb((A < B).astype(f32) * B))
        if eid == 6: return rb(rb(rb(rb(A + B) - A) * B) / A)
        if eid == 7: return A - f32(1.5)
        if eid == 8: return rb(f32(2) - A)
    raise ValueError(eid)


@pytest.mark.gpu
def test_api_bf16_expressions(api, g):
    n = 0
    while f"expr{n}_id" in g:
        eid = int(g[f"expr{n}_id"])
        a, b, want = g[f"expr{n}_a"], g[f"expr{n}_b"], g[f"expr{n}_out"]
        r, c = np.zeros(1, np.int32), np.zeros(1, np.int32)
        out = np.zeros(want.shape, np.float32)
        ok(api, api.api_bf16_expr(eid, fp(a), a.shape[0], a.shape[1], fp(b), b.shape[0], b.shape[1], fp(out), ip(r),
                                  ip(c)))
        assert (r[0], c[0]) == want.shape
        model = np.asarray(bf16_model(eid, a, b, *want.shape), np.float32)
        if eid in (3, 4):
            assert within_ulp(out, model), (n, eid)
        else:
            assert bitexact(out, model), (n, eid)
        if eid != 6:  # (a + b - a) cancels in bf16
            close(out, want, atol=BF_ATOL, rtol=BF_RTOL)
        n += 1
    assert n >= 13


@pytest.mark.gpu
def test_api_bf16_gemm_linear_softmax_reductions(api, g):
    A, B, want = g["gemm_a"], g["gemm_b"], g["gemm_c"]
    M, K = A.shape
    N = B.shape[1]
    C = np.zeros((M, N), np.float32)
    ok(api, api.api_bf16_gemm(M, N, K, fp(A), fp(B), fp(C)))
    exact = (rb(A).astype(np.float64) @ rb(B).astype(np.float64)).astype(np.float32)
    assert within_ulp(C, rb(exact))
    close(C, want, atol=BF_ATOL, rtol=BF_RTOL)

    W, b, X, want = g["linear_w"], g["linear_b"], g["linear_x"], g["linear_y"]
    Y = np.zeros_like(want)
    ok(api, api.api_bf16_linear(fp(W), fp(b), fp(X), W.shape[0], W.shape[1], X.shape[1], fp(Y)))
    prod = rb((rb(W).astype(np.float64) @ rb(X).astype(np.float64)).astype(np.float32))
    model = rb(prod + rb(b).reshape(-1, 1))
    assert np.all(np.abs(Y - model) <= 2.0 ** -6 * np.abs(model) + 1e-30)  # two roundings
    close(Y, want, atol=BF_ATOL, rtol=BF_RTOL)

    x = g["x"]
    R, Cc = x.shape
    Ys = np.zeros_like(x)
    ok(api, api.api_bf16_hsoftmax(fp(x), R, Cc, fp(Ys)))
    xb = rb(x)
    m = xb.max(1, keepdims=True)
    e = rb(np.exp(rb(xb - m)))
    s = np.zeros((R, 1), np.float32)
    for j in range(Cc):  # the row sum runs in float, column by column
        s[:, 0] = s[:, 0] + e[:, j]
    model = rb(e / rb(s))
    assert np.all(np.abs(Ys - model) <= 2.0 ** -6 * np.abs(model) + 1e-30)
    close(Ys, g["hsoftmax"], atol=1e-2, rtol=BF_RTOL)
    assert np.allclose(Ys.sum(1), 1.0, atol=3e-2)

    hs, vs, hm = np.zeros(R, np.float32), np.zeros(Cc, np.float32), np.zeros(R, np.float32)
    sc = np.zeros(2, np.float32)
    ok(api, api.api_bf16_reductions(fp(x), R, Cc, fp(hs), fp(vs), fp(hm), fp(sc)))
    rs = np.zeros(R, np.float32)
    for j in range(Cc):
        rs = rs + xb[:, j]
    cs = np.zeros(Cc, np.float32)
    for i in range(R):
        cs = cs + xb[i, :]
    assert bitexact(hs, rb(rs)) and bitexact(vs, rb(cs)) and bitexact(hm, xb.max(1))
    close(hs, g["hsum"].reshape(hs.shape), atol=BF_ATOL, rtol=BF_RTOL)
    assert sc[1] == xb.max()


def rope_entry(r, c, d):
    """jasmine's rotation table entry (mat_RoPE_t.hpp:113-131), float32 angle as val_type."""
    a = np.float32(c) / np.float32(np.power(10000.0, np.float32(r // 2) / np.float32(d)))
    a = float(np.float32(a))
    if r % 2 == c % 2:
        return math.cos(a)
    return math.sin(a) if r % 2 else -math.sin(a)


def test_api_rope_blocks(api):
    """mat_RoPE_t host blocks: forward_unite(1, 1) at d 4 is the closed form
    [cos .2, -sin .3; sin .2, cos .3] (angle c / 10000^((r/2)/d), 10000^(-1/4) = 0.1), and
    ragged range() requests (odd start, 3 x 5, 1 x 1) match the entry formula element by
    element.
    Host-only: no device work runs."""
    d = 4
    blk4 = np.zeros(4, np.float32)
    for (r0, R, c0, C) in ((1, 3, 3, 5), (2, 1, 7, 1), (0, 4, 0, 9)):
        blk = np.zeros(R * C, np.float32)
        ok(api, api.api_rope_blocks(d, 1, 1, fp(blk4), r0, R, c0, C, fp(blk)))
        a2, a3 = 2 / 10000 ** 0.25, 3 / 10000 ** 0.25
        assert np.allclose(blk4, [math.cos(a2), -math.sin(a3), math.sin(a2), math.cos(a3)], atol=1e-6)
        want = [[rope_entry(r0 + i, c0 + j, d) for j in range(C)] for i in range(R)]
        assert np.allclose(blk.reshape(R, C), want, atol=1e-6)
