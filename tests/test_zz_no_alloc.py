"""The allocation-free decode entry point (jas_attn_decode_noalloc) against jas_attn_decode.

Both run the same kernels; only where the split partials live differs (a static device array
against the caller's workspace), so the outputs must be bit-identical.  Two calls in a row,
the second with a smaller shape, check that the shared array carries nothing from one call
into the next; a shape whose partials exceed the array is rejected before any launch."""
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
    # first call: 16 x 32 heads of 128 over up to 2100 keys (3 splits); second: a smaller
    # shape (4 x 8 heads of 64, ragged lengths, more splits per pair) in the same array
    for B, H, D, lens, seed in ((16, 32, 128, [2100 - 37 * i for i in range(16)], 71),
                                (4, 8, 64, [900, 1, 333, 517], 72)):
        want, got = _decode_both(jas, B, H, D, lens, seed)
        assert np.isfinite(want).all()
        assert np.array_equal(got, want), f"B={B} H={H} D={D}: max diff {np.abs(got - want).max():.3g}"


def test_noalloc_decode_rejects_oversize(jas):
    from jasmine_amd import JasError
    B, H, D, ml = 16, 128, 128, 200000  # partials far beyond the static array
    assert jas.lib.jas_attn_decode_workspace(B, H, D, ml) > jas.lib.jas_attn_decode_scratch_max()
    with pytest.raises(JasError, match="scratch"):
        # null tensors: the size check comes first, nothing is launched
        jas.check(jas.lib.jas_attn_decode_noalloc(None, None, None, None, None, B, H, D, ml, 0, 0, 1.0, None))
