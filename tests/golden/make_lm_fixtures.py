"""Write tests/golden/lm_fixture_<case>.npz: greedy-decode fixtures of the decoder LMs at
the benchmark's own lengths, computed by the CPU oracle (oracle/liboracle.so,
``orc_lm_generate``).  TEST INFRASTRUCTURE ONLY.

The weights are built here on the host from the shared counter-based generator with the
same (seed, stream, index) assignment the device initialiser uses (``jas_lm_init_random``):
tensors are visited in name order, the k-th name (1-based) draws stream k, element
(l, r, c) of a [layers][rows][cols] tensor is index (l*rows + r)*cols + c, norm gains are 1
and biases 0.  Nothing here is read back from a GPU, so a fixture pins the device weight
generator, its RoPE table and its K/V rows at every position independently of the runner.

Each fixture holds the prompt row, the oracle's greedy ids of every decode step (the GPU
test feeds them back, teacher forcing), the two largest logits of every step (so a test
knows where an id is decided by more than its tolerance) and the full logits at a few steps.

    python tests/golden/make_lm_fixtures.py [case ...]     # default: every case

The config-5 cases stream 26 GB of fp32 weights per token through the scalar restatement:
about an hour each on 8 host cores.
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from oracle_lib import orc, fp, ip, randint, LmCfg, LmWeights, LM_WEIGHT_FIELDS  # noqa: E402

# name: (kind, n_layer, d, H, F, V, weight seed, batch of the bench prompt, prompt length,
#        prompt seed, sequence taken from that batch, decode steps, steps whose logits are kept)
CASES = {
    # config 4: GPT-2-small shape, bench batch 8 x 512 (seed 3), 256 greedy steps
    "config4_seq0": (0, 12, 768, 12, 3072, 50257, 3, 8, 512, 3, 0, 256, (0, 1, 2, 128, 255)),
    "config4_seq5": (0, 12, 768, 12, 3072, 50257, 3, 8, 512, 3, 5, 256, (0, 1, 2, 128, 255)),
    # config 5: LLaMA-7B shape, bench batch 16 x 2048 (seed 4), 128 greedy steps; the batch-1
    # bench line decodes sequence 0, sequence 11 stands for the batch-16 line
    "config5_seq0": (1, 32, 4096, 32, 11008, 32000, 4, 16, 2048, 4, 0, 128, (0, 1, 2, 64, 127)),
    "config5_seq11": (1, 32, 4096, 32, 11008, 32000, 4, 16, 2048, 4, 11, 128, (0, 1, 2, 64, 127)),
}


def tensor_shapes(kind, L, d, F, V, ctx):
    """(layers, rows, cols) of every weight tensor the runner holds, by name."""
    t = {"wte": (1, V, d), "ln1_g": (L, 1, d), "w_qkv": (L, 3 * d, d), "w_o": (L, d, d), "ln2_g": (L, 1, d),
         "lnf_g": (1, 1, d)}
    if kind == 0:
        t.update(wpe=(1, ctx, d), ln1_b=(L, 1, d), b_qkv=(L, 1, 3 * d), b_o=(L, 1, d), ln2_b=(L, 1, d),
                 w_fc=(L, F, d), b_fc=(L, 1, F), w_proj=(L, d, F), b_proj=(L, 1, d), lnf_b=(1, 1, d))
    else:
        t.update(w_gate=(L, F, d), w_up=(L, F, d), w_down=(L, d, F), w_head=(1, V, d))
    return t


def host_weights(kind, L, d, F, V, ctx, seed, std=0.02):
    """The runner's random initialisation, generated on the host."""
    out = {}
    for sid, (name, shp) in enumerate(sorted(tensor_shapes(kind, L, d, F, V, ctx).items()), start=1):
        n = int(np.prod(shp))
        a = np.empty(n, np.float32)
        if name in ("ln1_g", "ln2_g", "lnf_g"):
            a[:] = 1.0
        elif name[0] == "b" or name in ("ln1_b", "ln2_b", "lnf_b"):
            a[:] = 0.0
        else:
            orc.orc_fill_normal(fp(a), n, seed, sid, 0.0, std)
        out[name] = a
    return out


def make(case, nthreads=8):
    kind, L, d, H, F, V, seed, Bb, P, pseed, seq, steps, keep = CASES[case]
    ctx = P + steps
    prompt = np.ascontiguousarray(randint((Bb, P), V, pseed)[seq:seq + 1])
    w = host_weights(kind, L, d, F, V, ctx, seed)
    ocfg = LmCfg(kind, L, d, H, F, V, ctx, 1e-5 if kind == 0 else 1e-6, 10000.0, 0)
    ow = LmWeights(*[fp(w[n]) if n in w else None for n in LM_WEIGHT_FIELDS])
    ids = np.zeros((1, steps), np.int32)
    lg = np.zeros((steps, 1, V), np.float32)
    t0 = time.time()
    orc.orc_lm_generate(ocfg, ow, 1, P, ip(prompt), steps, None, ip(ids), fp(lg), nthreads)
    dt = time.time() - t0
    keep = np.array(keep, np.int32)
    top2 = np.sort(lg[:, 0], -1)[:, -2:]  # per step: runner-up and best logit
    path = os.path.join(HERE, f"lm_fixture_{case}.npz")
    np.savez_compressed(path, cfg=np.array([kind, L, d, H, F, V, seed, Bb, P, pseed, seq, steps], np.int64),
                        prompt=prompt[0], ids=ids[0], top2=top2, logit_steps=keep, logits=lg[keep, 0])
    print(f"{case}: {P}+{steps} tokens in {dt:.0f} s -> {path}", flush=True)


if __name__ == "__main__":
    nthreads = int(os.environ.get("ORC_THREADS", "8"))
    for c in sys.argv[1:] or list(CASES):
        make(c, nthreads)
