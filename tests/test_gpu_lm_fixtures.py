"""Decoder-LM runner against CPU-oracle fixtures at the benchmark's own lengths.

tests/golden/make_lm_fixtures.py ran the oracle (oracle/liboracle.so, orc_lm_generate) on
host-generated weights for the bench workloads: config 4 (GPT-2-small shape, 8 x 512-token
prompts, 256 greedy steps; sequences 0 and 5) and config 5 (LLaMA-7B shape, 16 x 2048-token
prompts, 128 greedy steps; sequence 0, which the batch-1 bench line decodes, and sequence
11 of the batch-16 line).  The GPU side initialises its own weights on the device from the
same generator and runs the bench's batch; the fixture's sequence is teacher-forced with the
oracle's ids, the other sequences run free.  This pins what a self-recompute check cannot:
the device weight generator, the RoPE table and the K/V rows at every position up to 2176.

Logits at the stored steps: |gpu - cpu| <= 1e-3 + 1e-4 |cpu|.  Greedy ids at every step must
match wherever the oracle's top-2 margin exceeds that tolerance (reference decode loop:
transformer_test.hpp:194-242).
"""
import glob
import os

import numpy as np
import pytest

from oracle_lib import randint

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "lm_fixture_*.npz")))
ATOL, RTOL = 1e-3, 1e-4


def load(path):
    f = np.load(path)
    kind, L, d, H, F, V, seed, Bb, P, pseed, seq, steps = (int(v) for v in f["cfg"])
    return dict(kind=kind, L=L, d=d, H=H, F=F, V=V, seed=seed, Bb=Bb, P=P, pseed=pseed, seq=seq, steps=steps,
                prompt=f["prompt"], ids=f["ids"], top2=f["top2"], logit_steps=f["logit_steps"], logits=f["logits"])


def test_fixtures_present():
    names = {os.path.basename(p) for p in FIXTURES}
    for c in ("config4_seq0", "config4_seq5", "config5_seq0", "config5_seq11"):
        assert f"lm_fixture_{c}.npz" in names, c


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[11:-4] for p in FIXTURES])
def test_fixture_self_consistent(path):
    """CPU: the stored prompt is the bench's prompt row (regenerated from its seed), each kept
    step's id is the argmax of its stored logits, and the stored top-2 agree with them."""
    f = load(path)
    assert np.array_equal(f["prompt"], randint((f["Bb"], f["P"]), f["V"], f["pseed"])[f["seq"]])
    for k, s in enumerate(f["logit_steps"]):
        lg = f["logits"][k]
        assert int(np.argmax(lg)) == int(f["ids"][s])
        assert np.array_equal(np.sort(lg)[-2:], f["top2"][s])
    assert f["ids"].shape == (f["steps"],) and np.all((f["ids"] >= 0) & (f["ids"] < f["V"]))


def _run(jas, lm, f, B):
    """Prefill the bench batch (B rows of the bench prompt), then decode f['steps'] - 1 steps;
    row f['seq'] (or row 0 when B == 1) is teacher-forced with the fixture's ids."""
    prompt = randint((f["Bb"], f["P"]), f["V"], f["pseed"])
    row = f["seq"] if B > 1 else 0
    prompt = prompt[f["seq"]:f["seq"] + 1] if B == 1 else prompt[:B]
    keep = {int(s): k for k, s in enumerate(f["logit_steps"])}
    nxt, lg = lm.prefill(prompt, want_logits=True)
    got_ids, got_lg = [int(nxt[row])], {0: lg[row].copy()}
    for s in range(1, f["steps"]):
        feed = nxt.copy()
        feed[row] = f["ids"][s - 1]
        nxt, lg = lm.decode(feed, want_logits=s in keep)
        got_ids.append(int(nxt[row]))
        if s in keep:
            got_lg[s] = lg[row].copy()
    for s, k in keep.items():
        want = f["logits"][k].astype(np.float64)
        err = np.abs(got_lg[s].astype(np.float64) - want)
        bad = err > ATOL + RTOL * np.abs(want)
        assert not bad.any(), f"step {s}: {bad.sum()} logits off, max abs err {err.max():.3g}"
    t1, t2 = f["top2"][:, 1].astype(np.float64), f["top2"][:, 0].astype(np.float64)
    decisive = (t1 - t2) > ATOL + RTOL * np.abs(t1)
    got_ids = np.array(got_ids)
    mism = np.nonzero(decisive & (got_ids != f["ids"]))[0]
    assert mism.size == 0, f"greedy ids differ at decisive steps {mism[:8]}"
    return int((~decisive).sum())


def _fixtures(prefix):
    return [p for p in FIXTURES if os.path.basename(p).startswith(f"lm_fixture_{prefix}")]


@pytest.mark.gpu
def test_config4_bench_batch_against_fixtures(jas):
    """Config 4 as bench.py runs it: GPT-2-small shape, ctx 1024, batch 8 of 512-token prompts,
    256 greedy steps; each fixture's sequence compared over the whole decode."""
    fs = [load(p) for p in _fixtures("config4")]
    if not fs:
        pytest.skip("no config-4 fixtures")
    cfg = jas.LmConfig(0, 12, 768, 12, 3072, 50257, 1024, 8, 1e-5, 10000.0)
    lm = jas.Lm(cfg)
    lm.init_random(fs[0]["seed"], 0.02)
    for f in fs:
        _run(jas, lm, f, 8)
    lm.close()


@pytest.mark.gpu
def test_config5_bench_batches_against_fixtures(jas):
    """Config 5 as bench.py runs it: LLaMA-7B shape, 32 layers, 2048-token prompts then 128
    greedy steps (positions up to 2175); sequence 0 at batch 1 (the batch-1 line) and
    sequence 11 inside the full batch of 16 (the headline line)."""
    fs = {os.path.basename(p)[11:-4]: load(p) for p in _fixtures("config5")}
    if not fs:
        pytest.skip("no config-5 fixtures")
    f0 = next(iter(fs.values()))
    cfg = jas.LmConfig(1, 32, 4096, 32, 11008, 32000, f0["P"] + f0["steps"], 16, 1e-6, 10000.0)
    lm = jas.Lm(cfg)
    lm.init_random(f0["seed"], 0.02)
    if "config5_seq0" in fs:
        _run(jas, lm, fs["config5_seq0"], 1)
    if "config5_seq11" in fs:
        _run(jas, lm, fs["config5_seq11"], 16)
    lm.close()


@pytest.mark.gpu
@pytest.mark.parametrize("kind", [0, 1])
def test_device_weights_match_host_generator(jas, kind):
    """The fixtures' host weights (make_lm_fixtures.host_weights) are the device
    initialiser's, bit for bit, at a small shape of each kind."""
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from make_lm_fixtures import host_weights
    L, d, H, F, V, ctx = 2, 128, 4, 208, 333, 40
    cfg = jas.LmConfig(kind, L, d, H, F, V, ctx, 2, 1e-5, 10000.0)
    lm = jas.Lm(cfg)
    lm.init_random(7, 0.02)
    hw = host_weights(kind, L, d, F, V, ctx, 7)
    for name, a in hw.items():
        assert np.array_equal(lm.weight(name).ravel(), a), name
    lm.close()
