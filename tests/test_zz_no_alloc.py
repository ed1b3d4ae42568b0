"""The allocation-free decode entry point (jas_attn_decode_noalloc) against jas_attn_decode.

Both run the same kernels; only where the split partials live differs (a static device array
against the caller's workspace), so the outputs must be bit-identical.  Two calls in a row,
the second with a smaller shape, check that the shared array carries nothing from one call
into the next; the array holds the partials of every shape."""
import math

import numpy as np
import pytest

from oracle_lib import normal

pytestmark = pytest.mark.gpu


def _decode_both(jas, B, H, D, lens, seed):
    ctx = max(lens) + 3
    K, V = normal((B, H, ctx, D), seed, 0), normal((B, H, ctx, D), seed, 1)
    q = normal((B, H, 1, D), seed, 2)
    sc = 1 / math.sqrt(D)
    dq, dk, dv = jas.to_device(q), jas.to_device(K), jas.to_device(V)
    dl = jas.to_device(np.array(lens, np.int32))
    ml = max(lens)
    ws_bytes = jas.lib.jas_attn_decode_workspace(B, H, D, ml)
    assert 0 < ws_bytes <= jas.lib.jas_attn_decode_scratch_max(), "shape must take the split path"
    ws = jas.DeviceArray(ws_bytes // 4)
    want, got = jas.DeviceArray((B, H, D)), jas.DeviceArray((B, H, D))
    jas.check(jas.lib.jas_attn_decode(dq.p, dk.p, dv.p, want.p, dl.p, B, H, D, ml, H * ctx * D, ctx * D, sc,
                                      ws.p, None))
    jas.check(jas.lib.jas_attn_decode_noalloc(dq.p, dk.p, dv.p, got.p, dl.p, B, H, D, ml, H * ctx * D, ctx * D, sc,
                                              None))
    return want.numpy(), got.numpy()


def test_noalloc_decode_matches_workspace_entry(jas):
    # first call: 4 x 32 heads of 128 over up to 2100 keys (4 splits); second: a smaller
    # shape (4 x 8 heads of 64, ragged lengths, more splits per pair) in the same array
    for B, H, D, lens, seed in ((4, 32, 128, [2100 - 370 * i for i in range(4)], 71),
                                (4, 8, 64, [900, 1, 333, 517], 72)):
        want, got = _decode_both(jas, B, H, D, lens, seed)
        assert np.isfinite(want).all()
        assert np.array_equal(got, want), f"B={B} H={H} D={D}: max diff {np.abs(got - want).max():.3g}"


def test_noalloc_scratch_covers_every_shape(jas):
    """The split count never asks for more than two to four workgroups per CU beyond the pairs
    themselves, so the partials of any shape stay below 1 MiB on this part and fit the
    static array (the entry point still checks the size and rejects a shape that would not)."""
    cap = jas.lib.jas_attn_decode_scratch_max()
    worst = 0
    for D in (32, 64, 128):
        for pairs in list(range(1, 130)) + [200, 255, 256, 257, 300, 384, 511, 512, 513, 1024, 4096]:
            for ml in (1, 100, 1000, 2300, 20000, 200000):
                worst = max(worst, jas.lib.jas_attn_decode_workspace(1, pairs, D, ml))
    assert 0 < worst <= cap, (worst, cap)
