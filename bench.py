"""Decode throughput of the LLaMA-7B-shaped fp32 decoder on one MI355X (config 5).

    python bench.py [--steps K] [--warmup W] [--batch 16] [--prompt 2048] [--no-gpt2] [--no-cpu]

Workload (config 5, the LLaMA-7B shape): 32 layers, d_model 4096, 32
heads (head dim 128), SwiGLU FFN 11008, RMSNorm eps 1e-6, RoPE theta 1e4, vocab 32000,
weights N(0, 0.02) from seed 4 (generated on the device), batch 16, prompts of 2048 token
ids uniform over the vocab (seed 4).  The prompt is prefilled (untimed, reported), W
greedy decode steps warm up, then K steps are timed; W + K <= 128 (the config's decode
length).  One step = one token for each of the 16 sequences through the whole model
(embedding, 32 layers, final norm, LM head, argmax) with the KV cache appended in place.

`value` comes from the K timed steps with no instrumentation.  The roofline object comes
from a second timed pass of K steps (positions right after the first) with HIP events
recorded around every launch on the runner's stream: per-launch events serialise the
queue and cost ~13% of step time, so they are kept out of the headline number.  cpu_baseline times the jasmine
reference itself (oracle/_ref, one host core) on one decode layer of one sequence at the real
shape and the LM-head GEMV, and extrapolates to a step of 16 sequences x 32 layers; cpu_configs
holds its config 2 / 3 timings.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, datasheet
FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix, datasheet
BF16_MFMA_TFLOPS = 2500.0  # MI355X dense bf16 matrix, datasheet


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def llama_cfg(jas, B, ctx, bf16=False):
    return jas.LmConfig(1, 32, 4096, 32, 11008, 32000, ctx, B, 1e-6, 10000.0, int(bf16), int(bf16))


def run_llama_bf16(jas, args):
    """The config-5 shape with bf16 weight and KV-cache storage (fp32 activations and
    accumulation).  Same prompt, warm-up and timed steps as
    the fp32 headline; returns its own line (not the headline value)."""
    from oracle_lib import randint
    B, P = args.batch, args.prompt
    L, d, H, F, V = 32, 4096, 32, 11008, 32000
    dh = d // H
    ctx = P + args.warmup + 2 * args.steps + 1
    lm = jas.Lm(llama_cfg(jas, B, ctx, bf16=True))
    if args.no_graph:
        lm.use_graph(False)
    lm.init_random(4, 0.02)
    lm.prefill(randint((B, P), V, 4))
    lm.generate(args.warmup, B)
    pos0 = lm.position
    jas.check(jas.lib.jas_synchronize(lm.stream))
    t0 = time.perf_counter()
    lm.generate(args.steps, B)
    dt = time.perf_counter() - t0
    pos1 = lm.position
    lm.profile(True)
    lm.generate(args.steps, B)
    ms, cnt = lm.profile(False)
    lm.close()
    w_step = 2 * (L * (4 * d * d + 3 * d * F) + V * d) + 4 * (2 * L + 1) * d
    kv_timed = sum(B * L * H * (pos0 + st + 1) * dh * 2 * 2 for st in range(args.steps)) / args.steps
    kv_prof = sum(B * L * H * (pos1 + st + 1) * dh * 2 * 2 for st in range(args.steps))
    step_bytes = w_step + kv_timed
    tok_s = B * args.steps / dt
    frac = step_bytes / (dt / args.steps) / 1e9 / HBM_PEAK_GBS
    gemm_gbs = (w_step - 4 * (2 * L + 1) * d) * args.steps / (ms[0] * 1e-3) / 1e9
    attn_gbs = kv_prof / (ms[1] * 1e-3) / 1e9
    log(f"[bench] llama bf16 storage: {tok_s:.1f} tok/s, {1e3 * dt / args.steps:.3f} ms/step, "
        f"{100 * frac:.1f}% of HBM peak (attention {attn_gbs:.0f} GB/s, weight GEMMs {gemm_gbs:.0f} GB/s)")
    return {"decode_tok_s": round(tok_s, 2), "ms_per_step": round(1e3 * dt / args.steps, 3),
            "step_bytes": step_bytes, "step_hbm_frac": round(frac, 4),
            "attention_gbs": round(attn_gbs, 1), "attention_frac": round(attn_gbs / HBM_PEAK_GBS, 4),
            "weight_gemm_gbs": round(gemm_gbs, 1), "weight_gemm_frac": round(gemm_gbs / HBM_PEAK_GBS, 4),
            "workload": f"config5 shape with bf16 weights and bf16 KV cache (fp32 activations and accumulation), "
                        f"batch {B}, {P}-token prompts, timed positions {pos0}..{pos0 + args.steps - 1}",
            "dtype": "bf16 storage / f32 compute"}


def weight_bytes_per_step(L, d, F, V):
    # every weight matrix is streamed once per decode step (embedding rows are gathered)
    return 4 * (L * (3 * d * d + d * d + 3 * d * F) + V * d)


def host_cpu():
    """Host CPU model and the logical CPUs this process may use."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return model, n


def cpu_baseline(B, ctx):
    """The reference CPU path (jasmine compiled from its own sources into oracle/_ref, -O2,
    one thread: the reference has no threading), timed on bounded samples at the real
    shapes and extrapolated:
      * one LLaMA-7B layer of one sequence's decode step over a `ctx`-key cache (seven
        weight_net_t::forward GEMVs, per-head mat_dot_t scores, hsoftmax, V P^T) and the
        32000 x 4096 LM-head GEMV; a step of B sequences costs B x (32 layers + head), since
        jasmine's mat_dot_t streams the weight once per output column;
      * config 2: the fused expression and hsoftmax at the full 8192^2;
      * config 3: one causal head (S 1024, D 64) of scores, mask, softmax and weighted sum,
        times the 96 heads.
    About 20 s of CPU work.  Returns (headline dict, per-config dict) or (None, None)."""
    import ctypes as C
    try:
        from oracle_lib import ref
    except Exception as e:  # pragma: no cover
        log("cpu baseline unavailable:", e)
        return None, None
    if ref is None:
        log("cpu baseline unavailable: oracle/_ref/libjasref.so not built")
        return None, None
    model, ncpu = host_cpu()
    attn = C.c_double()
    t_layer = ref.ref_time_llama_layer(4096, 32, 11008, ctx, C.byref(attn))
    t_head = ref.ref_time_linear(32000, 4096, 1, 1)
    step_s = B * (32 * t_layer + t_head)
    head = {"value": round(B / step_s, 6), "unit": "tok/s", "cores": 1, "kind": "reference",
            "host_cpu": model, "host_logical_cpus": ncpu,
            "sample": f"jasmine (oracle/_ref, g++ -O2, 1 thread) at the config-5 shape: one decode layer of one "
                      f"sequence over a {ctx}-key cache {t_layer:.2f} s (attention {attn.value:.2f} s), LM-head "
                      f"GEMV {t_head:.2f} s; extrapolated to a step of {B} sequences x 32 layers "
                      f"({step_s:.0f} s per step). jasmine itself has no KV cache: its decode loop recomputes the "
                      f"prefix, which at this context would cost a full prefill per token"}
    per = {}
    try:
        t_expr = ref.ref_time_cfg2(8192, 8192, 1)
        t_sm = ref.ref_time_hsoftmax(8192, 8192, 1)
        t_ah = ref.ref_time_attention_head(64, 1024)
        per = {"config2_expr_s": round(t_expr, 3), "config2_hsoftmax_s": round(t_sm, 3),
               "config2_expr_gbs": round(4 * 8192 * 8192 * 4 / t_expr / 1e9, 3),
               "config3_causal_attention_s": round(96 * t_ah, 2),
               "config3_note": "one head timed (scores, mask, hsoftmax, V P^T of mat_head_gen_t), x 96 heads",
               "config5_layer_s": round(t_layer, 3), "config5_lm_head_s": round(t_head, 3),
               "cores": 1, "host_cpu": model}
        per.update(cpu_more_configs(ref, ctx))
    except Exception as e:  # pragma: no cover
        log("[bench] cpu config lines failed:", e)
    return head, per


def cpu_more_configs(ref, ctx5):
    """The remaining CPU lines: config 1 timed in full through the restatement (jasmine has
    no GPT-2 block: pre-LN, GELU, learned positions), and sampled slices of configs 4 and 5
    through the reference's own objects (oracle/_ref), extrapolated and labelled so.  About
    15 s of one core."""
    import ctypes as C
    import numpy as np
    from oracle_lib import orc, fp, ip, normal, randint, LmCfg, LmWeights, LM_WEIGHT_FIELDS
    out = {}
    # config 1: 2 layers, d 128, 4 heads, FFN 512, vocab 256, 32-token prompt, 32 greedy steps
    L, d, H, F, V, P, S = 2, 128, 4, 512, 256, 32, 32
    shp = {"wte": (V, d), "wpe": (P + S, d), "ln1_g": (L, d), "ln1_b": (L, d), "w_qkv": (L, 3 * d, d),
           "b_qkv": (L, 3 * d), "w_o": (L, d, d), "b_o": (L, d), "ln2_g": (L, d), "ln2_b": (L, d),
           "w_fc": (L, F, d), "b_fc": (L, F), "w_proj": (L, d, F), "b_proj": (L, d), "lnf_g": (d,), "lnf_b": (d,)}
    w = {n: np.ascontiguousarray(normal(s, 0, k, 0.0, 0.02)) for k, (n, s) in enumerate(shp.items())}
    ow = LmWeights(*[fp(w[n]) if n in w else None for n in LM_WEIGHT_FIELDS])
    ids, prompt = np.zeros((1, S), np.int32), randint((1, P), V, 0)
    t0 = time.perf_counter()
    orc.orc_lm_generate(LmCfg(0, L, d, H, F, V, P + S, 1e-5, 1e4, 0), ow, 1, P, ip(prompt), S, None, ip(ids), None, 1)
    t1 = time.perf_counter() - t0
    out["config1_full_s"] = round(t1, 4)
    out["config1_tok_s"] = round(S / t1, 1)
    out["config1_note"] = ("timed in full (32-token prompt + 32 greedy steps, KV cache) through the C restatement "
                           "oracle/oracle.c, 1 thread: kind 'port', jasmine has no GPT-2 block")
    # config 4: GPT-2 small, batch 8, 512-token prompts, greedy decode at ~560 keys
    a = C.c_double()
    t_l4 = ref.ref_time_gpt2_layer(768, 12, 3072, 560, C.byref(a))
    t_h4 = ref.ref_time_linear(50257, 768, 1, 1)
    step4 = 8 * (12 * t_l4 + t_h4)
    ap = C.c_double()
    t_p4 = ref.ref_time_prefill_layer(0, 768, 12, 3072, 128, C.byref(ap))
    pf4 = 8 * 12 * ((t_p4 - ap.value) * 512 / 128 + ap.value * (512 / 128) ** 2)
    out.update(config4_layer_s=round(t_l4, 4), config4_layer_attention_s=round(a.value, 4),
               config4_lm_head_s=round(t_h4, 4), config4_step_s_extrapolated=round(step4, 3),
               config4_decode_tok_s_extrapolated=round(8 / step4, 3),
               config4_prefill_slice_s=round(t_p4, 3), config4_prefill_slice_attention_s=round(ap.value, 3),
               config4_prefill_s_extrapolated=round(pf4, 1),
               config4_note=("reference objects (oracle/_ref, g++ -O2, 1 thread): one GPT-2-small decode layer of "
                             "one sequence over 560 cached keys, the 50257 x 768 LM-head GEMV, and one layer of a "
                             "128-token prefill slice; extrapolated to 8 sequences x 12 layers (decode) and to "
                             "8 x 512-token prompts (projections x 4, attention x 16)"))
    # config 5 prefill slice: one layer over 4 tokens (projections; jasmine's mat_dot_t streams
    # the weights once per token column) and one causal head over 256 tokens (attention)
    t_p5 = ref.ref_time_prefill_layer(1, 4096, 32, 11008, 4, C.byref(ap))
    t_a5 = ref.ref_time_attention_head(128, 256)
    pf5 = 16 * 32 * ((t_p5 - ap.value) * 2048 / 4 + 32 * t_a5 * (2048 / 256) ** 2)
    out.update(config5_prefill_slice_s=round(t_p5, 3), config5_prefill_head256_s=round(t_a5, 4),
               config5_prefill_s_extrapolated=round(pf5, 0),
               config5_prefill_note=("reference objects: one LLaMA-7B layer's projections over a 4-token slice "
                                     "(x 512 tokens) and one causal head over 256 tokens (x 32 heads x 64 for "
                                     "2048 tokens), extrapolated to 16 x 2048-token prompts x 32 layers"))
    log(f"[bench] cpu: config1 {t1:.3f} s in full; config4 step {step4:.1f} s, prefill {pf4:.0f} s (extrapolated); "
        f"config5 prefill {pf5:.0f} s (extrapolated)")
    return out


def gpt2_decode_bytes(L, d, F, V, B, ctx):
    """HBM bytes of one GPT-2-style decode step: every weight matrix and bias once (the LM
    head is the tied embedding), plus K and V of the `ctx` cached positions per sequence."""
    weights = 4 * (L * (3 * d * d + d * d + 2 * d * F + 3 * d + d + F + d + 4 * d) + V * d + 2 * d)
    return weights + B * L * 2 * d * 4 * ctx


def run_gpt2(jas, cfg_args, B, P, seed, steps, warmup, graph=True):
    """Greedy decode of a GPT-2-style LM (configs 1 and 4); returns (tok/s, ms per step,
    HBM bytes per step at the timed steps' mean context)."""
    from oracle_lib import randint
    L, d, H, F, V, ctx = cfg_args
    cfg = jas.LmConfig(0, L, d, H, F, V, ctx, B, 1e-5, 10000.0)
    lm = jas.Lm(cfg)
    lm.use_graph(graph)
    lm.init_random(seed, 0.02)
    prompt = randint((B, P), V, seed)
    lm.prefill(prompt)  # first call: buffers and kernels warm
    t0 = time.perf_counter()
    lm.prefill(prompt)  # returns after the next ids are on the host
    prefill_s = time.perf_counter() - t0
    lm.generate(warmup, B)
    t0 = time.perf_counter()
    lm.generate(steps, B)
    dt = time.perf_counter() - t0
    lm.close()
    mean_ctx = P + warmup + (steps + 1) / 2.0
    # prefill flops: every projection of every prompt token, causal attention, the LM head
    # for the last position of each sequence
    pf = 2.0 * B * P * L * (4 * d * d + 2 * d * F) + 4.0 * B * L * (P * P / 2.0) * d + 2.0 * B * V * d
    run_gpt2.last_prefill = {"tok_s": round(B * P / prefill_s, 1), "ms": round(1e3 * prefill_s, 3),
                             "tflops": round(pf / prefill_s / 1e12, 2),
                             "mfma_frac": round(pf / prefill_s / 1e12 / FP32_MFMA_TFLOPS, 4)}
    return B * steps / dt, 1e3 * dt / steps, gpt2_decode_bytes(L, d, F, V, B, mean_ctx)


def read_ceiling():
    """Streaming-read rate of jas_hbm_read_probe (grid-stride nontemporal 16-byte loads, 8 in
    flight per thread, 256-thread workgroups) by transfer size and workgroup count.  'fresh':
    successive launches read successive ranges of a 1 GiB buffer, so a range is not re-read
    while the Infinity Cache could still hold it; 'same': every launch re-reads one range."""
    import ctypes as C
    import numpy as np
    import jasmine_amd as jas
    from jasmine_amd.timing import time_launches
    lib, chk = jas.lib, jas.check
    chk(lib.jas_init(0))
    n = 1 << 28
    buf = jas.DeviceArray((n,))
    chk(lib.jas_fill_normal(buf.p, n, 0, 0, 0.0, 1.0, None))
    sink = jas.DeviceArray((1,), np.uint32)
    out = {"unit": "GB/s (us per launch in brackets)", "fresh": {}, "same": {}}
    for nb in (2359296, 9437184, 50331648, 201326592):
        for wgs in (48, 96, 192, 256, 512, 2048):
            offs = iter([((i * nb) % ((1 << 30) - nb)) // 256 * 256 for i in range(4000)])
            ms = time_launches(lambda: chk(lib.jas_hbm_read_probe(C.c_void_p(buf.ptr + next(offs)), nb, wgs, 8, 1,
                                                                  sink.p, None)), 30)
            out["fresh"].setdefault(str(nb), {})[str(wgs)] = f"{nb / ms / 1e6:.0f} ({ms * 1e3:.2f})"
            ms = time_launches(lambda: chk(lib.jas_hbm_read_probe(buf.p, nb, wgs, 8, 1, sink.p, None)), 30)
            out["same"].setdefault(str(nb), {})[str(wgs)] = f"{nb / ms / 1e6:.0f} ({ms * 1e3:.2f})"
    print(json.dumps({"hbm_read_ceiling": out}, indent=1), flush=True)


def run_kernel_legs(jas, reps=10):
    """Configs 2 and 3 as per-kernel lines: HIP events on the library stream around `reps`
    back-to-back launches of each kernel at the config's full shape (inputs resident)."""
    import ctypes as C
    import numpy as np
    from jasmine_amd import expr as E
    from jasmine_amd.timing import time_launches
    lib, chk = jas.lib, jas.check
    out = {}

    # config 2: 8192 x 8192 fp32, A, B, C ~ N(0, 1) from seed 1
    R = Cc = 8192
    n = R * Cc
    A, Bm, Cm = (jas.DeviceArray((R, Cc)) for _ in range(3))
    for k, m in enumerate((A, Bm, Cm)):
        chk(lib.jas_fill_normal(m.p, n, 1, k, 0.0, 1.0, None))
    D, Y = jas.DeviceArray((R, Cc)), jas.DeviceArray((R, Cc))
    tree = E.leaf(A) * E.leaf(Bm) + 0.5 * E.leaf(Cm) - E.un("tanh", E.leaf(A))
    prog, leaves = E.lower(tree)
    from jasmine_amd.capi import Ins, Leaf
    pa = (Ins * len(prog))(*[Ins(o, d, a, 0, i) for o, d, a, i in prog])
    la = (Leaf * len(leaves))(*leaves)
    mb = n * 4

    def line(name, ms, bytes_, bound="hbm", flops=None, peak=None):
        if bound == "hbm":
            ach = bytes_ / (ms * 1e-3) / 1e9
            return {"kernel": name, "avg_launch_us": round(ms * 1e3, 2), "bound": "hbm", "bytes": bytes_,
                    "achieved": round(ach, 1), "unit": "GB/s", "peak": HBM_PEAK_GBS, "frac": round(ach / HBM_PEAK_GBS, 4)}
        ach = flops / (ms * 1e-3) / 1e12
        return {"kernel": name, "avg_launch_us": round(ms * 1e3, 2), "bound": "mfma", "flops": flops,
                "achieved": round(ach, 2), "unit": "TFLOP/s", "peak": peak, "frac": round(ach / peak, 4)}

    # the achievable-bandwidth reference for the HBM-bound lines: the runtime's own
    # device-to-device copy of one 8192^2 fp32 matrix (one read and one write per byte)
    ms = time_launches(lambda: chk(lib.jas_memcpy_d2d(D.p, A.p, mb, None)), reps)
    out["hbm_copy"] = line("device-to-device copy (HIP runtime), 268 MB: achievable-bandwidth reference", ms, 2 * mb)
    # the achievable streaming-read rate (jas_hbm_read_probe: grid-stride nontemporal 16-byte
    # reads, 8 in flight per thread) at two of the decode kernels' sizes: config 3's 50 MB
    # K/V and a 201 MB LLaMA-7B QKV matrix, read from the 268 MB matrix A
    big = A
    sink = jas.DeviceArray((1,), np.uint32)
    ceil = {}
    for nb in (50331648, 201326592):
        ms = time_launches(lambda: chk(lib.jas_hbm_read_probe(big.p, nb, 2048, 8, 1, sink.p, None)), reps * 3)
        ceil[str(nb)] = round(nb / (ms * 1e-3) / 1e9, 1)
    out["hbm_read_ceiling"] = {"kernel": "read_probe_kernel<8, nontemporal> (jas_hbm_read_probe), 2048 x 256 threads",
                               "GB_s_by_bytes": ceil, "peak": HBM_PEAK_GBS,
                               "note": "repeated reads of one buffer (the Infinity Cache may hold the 50 MB case)"}
    ms = time_launches(lambda: chk(lib.jas_ew_eval(pa, len(prog), la, len(leaves), D.p, 0, R, Cc, None)), reps)
    out["ew_cfg2"] = line("ew_eval_kernel: D = A*B + 0.5*C - tanh(A), 8192^2 fp32 (3 reads + 1 write)", ms, 4 * mb)
    ms = time_launches(lambda: chk(lib.jas_softmax(D.p, Y.p, R, Cc, Cc, Cc, 1, None)), reps)
    out["softmax_rows"] = line("row softmax, 8192 rows of 8192", ms, 2 * mb)
    ms = time_launches(lambda: chk(lib.jas_layernorm(D.p, Y.p, R, Cc, Cc, Cc, 1, C.c_float(1e-5), None, None, None)),
                       reps)
    out["layernorm_rows"] = line("row LayerNorm eps 1e-5, 8192 rows of 8192", ms, 2 * mb)
    ms = time_launches(lambda: chk(lib.jas_rmsnorm(D.p, Y.p, R, Cc, Cc, Cc, 1, C.c_float(1e-6), None, None)), reps)
    out["rmsnorm_rows"] = line("row RMSNorm eps 1e-6, 8192 rows of 8192", ms, 2 * mb)
    del A, Bm, Cm, D, Y

    # config 3: causal attention B=8, H=12, S=1024, D=64, Q, K, V ~ N(0, 1) from seed 2
    Bb, H, S, Dh = 8, 12, 1024, 64
    shape, ne = (Bb, H, S, Dh), Bb * H * S * Dh
    Q, K, V, O = (jas.DeviceArray(shape) for _ in range(4))
    for k, m in enumerate((Q, K, V)):
        chk(lib.jas_fill_normal(m.p, ne, 2, k, 0.0, 1.0, None))
    st = (H * S * Dh, S * Dh, Dh)
    causal_flops = 4.0 * Bb * H * S * S * Dh / 2

    def prefill(q, k, v, o, dt):
        chk(lib.jas_attn_prefill(q.p, k.p, v.p, o.p, Bb, H, S, S, Dh, *st, *st, *st, C.c_float(0.125), 1, dt, None))

    ms = time_launches(lambda: prefill(Q, K, V, O, 0), reps)
    out["attn_prefill_f32"] = line("flash_prefill_kernel<64> fp32 causal, B8 H12 S1024 D64", ms, None, "mfma",
                                   causal_flops, FP32_MFMA_TFLOPS)

    def bf(x):
        u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    Qb, Kb, Vb = (jas.to_device(bf(m.numpy())) for m in (Q, K, V))
    Ob = jas.DeviceArray(shape, np.uint16)
    ms = time_launches(lambda: prefill(Qb, Kb, Vb, Ob, 3), reps)
    out["attn_prefill_bf16"] = line("flash_prefill_kernel<64> bf16 in / fp32 accumulate, causal, same shape", ms, None,
                                    "mfma", causal_flops, BF16_MFMA_TFLOPS)
    del Qb, Kb, Vb, Ob

    q = jas.DeviceArray((Bb, H, Dh))
    chk(lib.jas_fill_normal(q.p, Bb * H * Dh, 2, 3, 0.0, 1.0, None))
    o = jas.DeviceArray((Bb, H, Dh))
    lens = jas.to_device(np.full(Bb, S, np.int32))
    ws = jas.DeviceArray(max(lib.jas_attn_decode_workspace(Bb, H, Dh, S) // 4, 1))
    ms = time_launches(lambda: chk(lib.jas_attn_decode(q.p, K.p, V.p, o.p, lens.p, Bb, H, Dh, S, st[0], st[1],
                                                       C.c_float(0.125), ws.p, None)), reps * 5)
    out["attn_decode_f32"] = line("attn_decode_kernel<64> (key splits merged by each pair's last split), 1 query over 1024 cached keys, B8 H12",
                                  ms, 2 * ne * 4)
    del Q, K, V, O

    # mat_dot_t / weight_net_t products (mat_express_t.hpp:730-736): row-major fp32 A [M][K]
    # times B [K][N] into C [M][N], on gemm_dma_kernel
    for nn in (1024, 4096):
        Ga, Gb, Gc = (jas.DeviceArray((nn, nn)) for _ in range(3))
        chk(lib.jas_fill_normal(Ga.p, nn * nn, 5, 0, 0.0, 1.0, None))
        chk(lib.jas_fill_normal(Gb.p, nn * nn, 5, 1, 0.0, 1.0, None))
        ms = time_launches(lambda: chk(lib.jas_gemm(nn, nn, nn, Ga.p, nn, 1, Gb.p, nn, 1, Gc.p, nn, 1, None, 0, 0, 0,
                                                    1, 0, 0, 0, 0, None)), reps * 2)
        out[f"gemm_{nn}"] = line(f"gemm_dma_kernel fp32, row-major {nn}^3 (mat_dot_t)", ms, None, "mfma",
                                 2.0 * nn ** 3, FP32_MFMA_TFLOPS)
        del Ga, Gb, Gc
    return out


# ---------------------------------------------------------------- rocprofv3 summaries
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "llama7b_decode_b16_traffic.json")
KCLASS = {"attention": ("attn_decode_kernel<128,",)}


def _pmc_per_kernel(csv_path, counter):
    """{kernel name: [value per dispatch]} for one derived counter of a rocprofv3 --pmc run."""
    import csv
    per = {}
    for r in csv.DictReader(open(csv_path)):
        if r["Counter_Name"] != counter:
            continue
        per.setdefault(r["Kernel_Name"], {}).setdefault(r["Dispatch_Id"], 0.0)
        per[r["Kernel_Name"]][r["Dispatch_Id"]] += float(r["Counter_Value"])
    return {k: list(v.values()) for k, v in per.items()}


def _pmc_dispatches(fetch_csv, write_csv, pattern):
    """[(FETCH_SIZE, WRITE_SIZE, kernel name)] per dispatch of kernels matching `pattern`, in
    dispatch order (the two runs launch the same sequence)."""
    import csv
    def per(path, counter):
        d = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter and pattern in r["Kernel_Name"]:
                k = int(r["Dispatch_Id"])
                d.setdefault(k, [0.0, r["Kernel_Name"]])
                d[k][0] += float(r["Counter_Value"])
        return [d[k] for k in sorted(d)]
    f, w = per(fetch_csv, "FETCH_SIZE"), per(write_csv, "WRITE_SIZE")
    return [(a[0], b[0], a[1]) for a, b in zip(f, w)]


def summarize_pmc(fetch_csv, write_csv, cfetch_csv, cwrite_csv, args):
    """HBM traffic per decode launch from FETCH_SIZE / WRITE_SIZE runs of this bench,
    calibrated by the same counters on a plain device copy of COPY_BYTES."""
    import numpy as np
    f, w = _pmc_per_kernel(fetch_csv, "FETCH_SIZE"), _pmc_per_kernel(write_csv, "WRITE_SIZE")
    cf, cw = _pmc_per_kernel(cfetch_csv, "FETCH_SIZE"), _pmc_per_kernel(cwrite_csv, "WRITE_SIZE")
    copy = [k for k in cf if "copyBuffer" in k or "copy" in k.lower()]
    kib = COPY_BYTES / 1024.0
    fcal = kib / np.median(cf[copy[0]]) if copy else 1.0
    wcal = kib / np.median(cw[copy[0]]) if copy else 1.0
    out = {"fetch_scale": fcal, "write_scale": wcal, "copy_bytes": COPY_BYTES, "classes": {}}
    for cls, pats in KCLASS.items():
        tot, n = 0.0, None
        for k in f:
            if any(pt in k for pt in pats):
                fk, wk = f[k], w.get(k, [0.0])
                tot += (np.mean(fk) * fcal + np.mean(wk) * wcal) * 1024.0 * len(fk)
                if pats[0] in k:
                    n = (n or 0) + len(fk)
        if n:
            out["classes"][cls] = {"bytes_per_launch": tot / n, "launches": n}
    # the skinny dispatches come in PROJ_ORDER, five each
    sk = _pmc_dispatches(fetch_csv, write_csv, "skinny_kernel<")
    per = {}
    for i, (name, K, M) in enumerate(PROJ_ORDER):
        rows = sk[5 * i:5 * i + 5]
        if len(rows) == 5:
            fb = np.mean([r[0] for r in rows]) * fcal * 1024.0
            wb = np.mean([r[1] for r in rows]) * wcal * 1024.0
            alg = 4.0 * M * K * (2 if name == "w_gate_up" else 1)
            per[name] = {"fetch_bytes": fb, "write_bytes": wb, "weight_bytes": alg, "ratio": (fb + wb) / alg,
                         "kernel": rows[0][2]}
    out["weight_gemms"] = per
    if per:
        tot = sum(v["fetch_bytes"] + v["write_bytes"] for v in per.values())
        alg = sum(v["weight_bytes"] for v in per.values())
        out["classes"]["weight_gemm"] = {"bytes_per_launch": tot / len(per), "launches": 5 * len(per)}
    B, H, dh = args.batch, 32, 128
    out["algorithmic"] = {"attention": B * H * profiled_mean_ctx(args) * dh * 8,
                          "weight_gemm": (sum(v["weight_bytes"] for v in per.values()) / len(per)) if per else None}
    out["run"] = {"batch": B, "prompt": args.prompt, "steps": args.steps, "warmup": args.warmup}
    out["shape"] = {"batch": B, "heads": H, "head_dim": dh, "kv": "f32"}
    out["mean_ctx"] = profiled_mean_ctx(args)
    return out


COPY_BYTES = 1 << 30


def profiled_mean_ctx(args):
    """Mean number of cached keys per decode step over the bench's profiled pass (positions
    P + warmup + steps .. P + warmup + 2 steps - 1; step s attends to position + 1 keys)."""
    pos1 = args.prompt + args.warmup + args.steps
    return pos1 + (args.steps + 1) / 2.0


# (jas_lm_project name, K, M) of the LLaMA-7B decode weight GEMMs, in launch order; weight
# bytes = 4 * M * K (gate_up: both matrices)
PROJ_ORDER = [("w_qkv", 4096, 3 * 4096), ("w_o", 4096, 4096), ("w_gate_up", 4096, 11008), ("w_down", 11008, 4096),
              ("w_head", 4096, 32000)]


def traffic_kernels(args):
    """The dominant decode kernel alone for rocprofv3 --pmc: the split-K attention at the
    LLaMA-7B shape (batch x 32 heads x 128) over the profiled pass's mean context (half the
    sequences one key shorter when the mean is a half), five launches.  Same kernels, same
    bytes per launch as inside the decode step; the runner itself is not profiled this way
    because rocprofv3's counter collection dies in the runner's launch path (host SIGSEGV)."""
    import ctypes as C
    import numpy as np
    import jasmine_amd as jas
    lib = jas.lib
    jas.check(lib.jas_init(0))
    B, H, D = args.batch, 32, 128
    mc = profiled_mean_ctx(args)
    lo = int(mc)
    lens_h = np.array([lo + (1 if (mc - lo) > 0 and b % 2 else 0) for b in range(B)], np.int32)
    # the runner's K/V cache rows are max_len long and it launches over its full capacity
    # (the splits past a sequence are empty): same strides and launch here
    max_len = args.prompt + args.warmup + 2 * args.steps + 1
    Kc, Vc = jas.DeviceArray((B, H, max_len, D)), jas.DeviceArray((B, H, max_len, D))
    jas.check(lib.jas_fill_normal(Kc.p, B * H * max_len * D, 5, 0, 0.0, 1.0, None))
    jas.check(lib.jas_fill_normal(Vc.p, B * H * max_len * D, 5, 1, 0.0, 1.0, None))
    q, o = jas.DeviceArray((B, H, D)), jas.DeviceArray((B, H, D))
    jas.check(lib.jas_fill_normal(q.p, B * H * D, 5, 2, 0.0, 1.0, None))
    lens = jas.to_device(lens_h)
    ws = jas.DeviceArray(max(lib.jas_attn_decode_workspace(B, H, D, max_len) // 4, 1))
    for _ in range(5):
        jas.check(lib.jas_attn_decode(q.p, Kc.p, Vc.p, o.p, lens.p, B, H, D, max_len, H * max_len * D, max_len * D,
                                      C.c_float(D ** -0.5), ws.p, None))
    jas.check(lib.jas_synchronize(None))
    del Kc, Vc
    # the decode weight GEMMs of one LLaMA-7B-width layer and the LM head, through
    # jas_lm_project: the decode step's own skinny_kernel variants on the runner's packed
    # weights, each launched five times in this order (pack_tokens_kernel and, for the split
    # projections, sum_splits_kernel go with each launch)
    lm = jas.Lm(llama_cfg(jas, B, 64))
    lm.init_random(4, 0.02)
    order = []
    for name, K, M in PROJ_ORDER:
        x, y = jas.DeviceArray((B, K)), jas.DeviceArray((B, M))
        jas.check(lib.jas_fill_normal(x.p, B * K, 5, 3, 0.0, 1.0, None))
        for _ in range(5):
            lm.project(name, 0, x, y, B)
        order.append(name)
    jas.check(lib.jas_synchronize(None))
    lm.close()
    print(json.dumps({"traffic_kernels": ["attn_decode"] + order, "batch": B, "heads": H, "head_dim": D,
                      "mean_ctx": float(lens_h.mean()), "launches": 5}))


def traffic_bf16_projections(args):
    """The decode weight GEMMs of the bf16-storage variant alone (for rocprofv3 counter runs):
    a LLaMA-7B-shape model with bf16 weights, each projection of layer 0 and the LM head
    through jas_lm_project, five launches each, in PROJ_ORDER."""
    import jasmine_amd as jas
    lib = jas.lib
    jas.check(lib.jas_init(0))
    B = args.batch
    lm = jas.Lm(llama_cfg(jas, B, 64, bf16=True))
    lm.init_random(4, 0.02)
    for name, K, M in PROJ_ORDER:
        x, y = jas.DeviceArray((B, K)), jas.DeviceArray((B, M))
        jas.check(lib.jas_fill_normal(x.p, B * K, 5, 3, 0.0, 1.0, None))
        for _ in range(5):
            lm.project(name, 0, x, y, B)
    jas.check(lib.jas_synchronize(None))
    lm.close()
    print(json.dumps({"traffic_bf16_projections": [n for n, _, _ in PROJ_ORDER], "batch": B, "launches": 5}))


def copy_calibration():
    """A plain device-to-device copy of COPY_BYTES (the copy-kernel reference for FETCH_SIZE /
    WRITE_SIZE), five times."""
    import jasmine_amd as jas
    jas.check(jas.lib.jas_init(0))
    a, b = jas.DeviceArray(COPY_BYTES // 4), jas.DeviceArray(COPY_BYTES // 4)
    a.zero()
    for _ in range(5):
        jas.check(jas.lib.jas_memcpy_d2d(b.p, a.p, COPY_BYTES, None))
    jas.check(jas.lib.jas_synchronize(None))
    print(json.dumps({"copy_calibration_bytes": COPY_BYTES, "repeats": 5}))


def load_traffic(args, dom_kernel_class, bytes_per_launch):
    """Measured HBM bytes per launch of the dominant class, scaled to this run.  The committed
    summary holds FETCH_SIZE + WRITE_SIZE per launch for a counter run of the same kernels at
    the same per-launch shape (batch, heads, head dim, cache element type) and its algorithmic
    bytes; the measured/algorithmic ratio is applied to this run's algorithmic bytes per
    launch (the context length only scales both).  None if no summary matches the shape."""
    try:
        t = json.load(open(TRAFFIC_FILE))
    except (OSError, ValueError):
        return None, None
    shape = t.get("shape", {})
    if shape != {"batch": args.batch, "heads": 32, "head_dim": 128, "kv": "f32"}:
        return None, None
    c = t.get("classes", {}).get(dom_kernel_class)
    alg = (t.get("algorithmic") or {}).get(dom_kernel_class)
    if c is None or not alg:
        return None, None
    ratio = c["bytes_per_launch"] / alg
    basis = (f"{TRAFFIC_FILE.split(os.sep)[-1]}: rocprofv3 FETCH_SIZE + WRITE_SIZE of the {dom_kernel_class} "
             f"kernels at this launch shape, mean context {t.get('mean_ctx')}, measured/algorithmic "
             f"{ratio:.4f}, applied to this run's bytes per launch")
    return round(ratio * bytes_per_launch), basis


def encdec_flops(d, H, ne, nd, T):
    """FLOPs of one encoder_forward and of one decoder forward (cross-attention keys/values
    already cached) of jasmine's transformer_base_t: per-head d_h x d_h projections, d x d
    output projection and FFN, attention 4*T*T*d (halved under the causal mask)."""
    dh = d // H
    mha_proj = 2.0 * 3 * d * dh * T + 2.0 * d * d * T
    ffn = 2.0 * d * d * T
    enc = ne * (mha_proj + 4.0 * T * T * d + ffn)
    dec = nd * (mha_proj + 2.0 * T * T * d + 2.0 * d * dh * T + 2.0 * d * d * T + 4.0 * T * T * d + ffn)
    return enc, dec


def run_encdec(reps=5):
    """jasmine's encoder-decoder transformer through the C++ API (tests/cpp/api_driver.cpp,
    built against this build's headers): wall ms per encoder_forward and per decoder forward,
    all-heads fused path and the per-head path (materialised scores)."""
    import ctypes as C
    path = os.path.join(ROOT, "tests", "cpp", "libjasapi.so")
    if not os.path.exists(path):
        return {"skipped": "tests/cpp/libjasapi.so is not built"}
    api = C.CDLL(path)
    api.api_last_error.restype = C.c_char_p
    out = {}
    for tag, (d, H, ne, nd, T) in {"base_T512": (512, 8, 6, 6, 512), "d1024_T1024": (1024, 16, 6, 6, 1024)}.items():
        fe, fd = encdec_flops(d, H, ne, nd, T)
        row = {"workload": f"transformer_base_t d {d}, {H} heads, {ne}+{nd} layers, {T} tokens in and out, fp32"}
        for fused in (1, 0):
            a, b = C.c_double(), C.c_double()
            rc = api.api_transformer_bench(d, H, ne, nd, T, T, fused, reps, C.byref(a), C.byref(b))
            if rc:
                raise RuntimeError(api.api_last_error().decode())
            row["fused" if fused else "per_head"] = {
                "encode_ms": round(a.value, 3), "forward_ms": round(b.value, 3),
                "encode_tflops": round(fe / a.value / 1e9, 2), "forward_tflops": round(fd / b.value / 1e9, 2)}
        row["mfma_frac_forward"] = round(row["fused"]["forward_tflops"] / 157.3, 4)
        out[tag] = row
        log(f"[bench] encdec {tag}: fused {row['fused']}, per-head {row['per_head']}")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=120)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--no-gpt2", action="store_true")
    ap.add_argument("--gpt2-only", action="store_true",
                    help="only the GPT-2-small (config 4) leg: 8 x 512 prefill, 4 + 32 decode steps")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-encdec", action="store_true", help="skip the C++ API encoder-decoder leg")
    ap.add_argument("--encdec-only", action="store_true",
                    help="only the C++ API encoder-decoder leg (one JSON object; for profilers)")
    ap.add_argument("--no-bf16", action="store_true", help="skip the bf16-storage LLaMA leg")
    ap.add_argument("--no-batch1", action="store_true", help="skip the batch-1 LLaMA leg")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the config 2/3 kernel lines (one JSON object; for profilers)")
    ap.add_argument("--no-kernels", action="store_true", help="skip the config 2/3 kernel lines")
    ap.add_argument("--no-graph", action="store_true",
                    help="decode with eager launches instead of graph replay (same kernels; for profilers)")
    ap.add_argument("--copy-calib", action="store_true", help="only run the copy used to calibrate PMC bytes")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="only the streaming-read sweep (jas_hbm_read_probe): sizes x workgroup counts, each "
                         "launch at a fresh offset of a 1 GiB buffer, plus re-reads of one buffer")
    ap.add_argument("--traffic-kernels", action="store_true",
                    help="only run the dominant decode kernel at the profiled pass's shape (for rocprofv3 --pmc)")
    ap.add_argument("--traffic-bf16", action="store_true",
                    help="only run the bf16-weight decode projections (for rocprofv3 counter runs)")
    ap.add_argument("--summarize-pmc", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV", "COPY_WRITE_CSV"),
                    help="write the traffic summary from rocprofv3 --pmc counter_collection.csv files")
    args = ap.parse_args()
    if args.copy_calib:
        copy_calibration()
        return
    if args.read_ceiling:
        read_ceiling()
        return
    if args.traffic_kernels:
        traffic_kernels(args)
        return
    if args.traffic_bf16:
        traffic_bf16_projections(args)
        return
    if args.kernels_only:
        import jasmine_amd as jas
        jas.check(jas.lib.jas_init(0))
        print(json.dumps({"kernels": run_kernel_legs(jas)}), flush=True)
        return
    if args.gpt2_only:
        import jasmine_amd as jas
        jas.check(jas.lib.jas_init(0))
        g_tok, g_ms, g_bytes = run_gpt2(jas, (12, 768, 12, 3072, 50257, 1024), 8, 512, 3, 32, 4,
                                        graph=not args.no_graph)
        print(json.dumps({"gpt2_small": {"decode_tok_s": round(g_tok, 1), "ms_per_step": round(g_ms, 3),
                                         "step_hbm_frac": round(g_bytes / (g_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                         "graph": not args.no_graph, "prefill": run_gpt2.last_prefill}}), flush=True)
        return
    if args.encdec_only:
        import jasmine_amd as jas
        jas.check(jas.lib.jas_init(0))
        print(json.dumps({"encdec_cpp_api": run_encdec()}), flush=True)
        return
    if args.summarize_pmc:
        out = summarize_pmc(*args.summarize_pmc, args)
        print(json.dumps(out, indent=1))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import jasmine_amd as jas
    from oracle_lib import randint

    os.environ.setdefault("JAS_VERBOSE", "1")
    jas.check(jas.lib.jas_init(0))
    kernels = None
    if not args.no_kernels:
        log("[bench] config 2/3 kernel lines")
        kernels = run_kernel_legs(jas)
        for k, v in kernels.items():
            if "avg_launch_us" in v:
                log(f"[bench]   {k}: {v['avg_launch_us']} us, {v['achieved']} {v['unit']} ({100 * v['frac']:.1f}% of peak)")
            else:
                log(f"[bench]   {k}: {v}")
    B, P = args.batch, args.prompt
    L, d, H, F, V = 32, 4096, 32, 11008, 32000
    dh = d // H
    ctx = P + args.warmup + 2 * args.steps + 1  # timed pass + profiled pass
    cfg = llama_cfg(jas, B, ctx)
    log(f"[bench] creating LLaMA-7B-shape fp32 model, batch {B}, ctx {ctx}")
    lm = jas.Lm(cfg)
    if args.no_graph:
        lm.use_graph(False)
    t0 = time.perf_counter()
    lm.init_random(4, 0.02)
    log(f"[bench] weights initialised in {time.perf_counter() - t0:.1f} s")
    prompt = randint((B, P), V, 4)
    t0 = time.perf_counter()
    lm.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    log(f"[bench] prefill {B}x{P} tokens: {prefill_s:.2f} s ({B * P / prefill_s:.0f} tok/s)")

    lm.generate(args.warmup, B)
    pos0 = lm.position
    jas.check(jas.lib.jas_synchronize(lm.stream))
    t0 = time.perf_counter()
    lm.generate(args.steps, B)  # synchronises at the end
    dt = time.perf_counter() - t0
    tok_s = B * args.steps / dt
    log(f"[bench] decode: {args.steps} steps in {dt:.3f} s -> {tok_s:.1f} tok/s")
    # profiled pass: HIP events around every launch on the runner's stream
    pos1 = lm.position
    lm.profile(True)
    t0 = time.perf_counter()
    lm.generate(args.steps, B)
    dt_prof = time.perf_counter() - t0
    ms, cnt = lm.profile(False)
    log(f"[bench] profiled pass: {args.steps} steps in {dt_prof:.3f} s; gpu ms by class {ms}, launches {cnt}")

    # algorithmic bytes over the profiled region
    w_bytes = weight_bytes_per_step(L, d, F, V) * args.steps
    kv_bytes = sum(B * L * H * (pos1 + s + 1) * dh * 4 * 2 for s in range(args.steps))
    step_bytes_timed = weight_bytes_per_step(L, d, F, V) + sum(
        B * L * H * (pos0 + s + 1) * dh * 4 * 2 for s in range(args.steps)) / args.steps
    gemm_gbs = w_bytes / (ms[0] * 1e-3) / 1e9
    attn_gbs = kv_bytes / (ms[1] * 1e-3) / 1e9
    step_bytes = (w_bytes + kv_bytes) / args.steps
    classes = [
        {"kernel": "skinny_kernel (decode weight GEMMs: QKV+RoPE+KV append, O+residual, SwiGLU, down+residual, LM head)",
         "achieved": gemm_gbs, "launches": cnt[0], "gpu_ms": ms[0], "bytes": w_bytes, "cls": "weight_gemm"},
        {"kernel": "attn_decode_kernel (KV-cache attention, one pass per (sequence, head) at 16 x 32 pairs)",
         "achieved": attn_gbs, "launches": cnt[1], "gpu_ms": ms[1], "bytes": kv_bytes, "cls": "attention"},
    ]
    dom = max(classes, key=lambda c: c["gpu_ms"])
    other = min(classes, key=lambda c: c["gpu_ms"])
    roof = {"bound": "hbm", "achieved": round(dom["achieved"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dom["achieved"] / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(args, dom["cls"], dom["bytes"] / max(dom["launches"], 1))[0],
            "traffic_basis": load_traffic(args, dom["cls"], dom["bytes"] / max(dom["launches"], 1))[1],
            "kernel": dom["kernel"],
            "bytes_per_launch": dom["bytes"] / max(dom["launches"], 1),
            "avg_launch_us": 1e3 * dom["gpu_ms"] / max(dom["launches"], 1)}
    step_roofline_frac = (step_bytes_timed / (dt / args.steps)) / 1e9 / HBM_PEAK_GBS

    # batch-1 decode on the same model (BASELINE's second config-5 row): re-prefill one sequence
    b1 = None
    try:
        if args.no_batch1:
            raise RuntimeError("skipped (--no-batch1)")
        lm.prefill(prompt[:1])
        lm.generate(args.warmup, 1)
        b1_pos0 = lm.position
        jas.check(jas.lib.jas_synchronize(lm.stream))
        t0 = time.perf_counter()
        lm.generate(args.steps, 1)
        b1_dt = time.perf_counter() - t0
        b1_bytes = weight_bytes_per_step(L, d, F, V) + sum(
            L * H * (b1_pos0 + st + 1) * dh * 4 * 2 for st in range(args.steps)) / args.steps
        b1_frac = b1_bytes / (b1_dt / args.steps) / 1e9 / HBM_PEAK_GBS
        b1 = {"decode_tok_s": round(args.steps / b1_dt, 2), "ms_per_step": round(1e3 * b1_dt / args.steps, 3),
              "step_bytes": b1_bytes, "step_hbm_frac": round(b1_frac, 4),
              "workload": f"config5 shape fp32, batch 1, {P}-token prompt, timed positions "
                          f"{b1_pos0}..{b1_pos0 + args.steps - 1}"}
        log(f"[bench] llama batch 1: {args.steps / b1_dt:.1f} tok/s, {1e3 * b1_dt / args.steps:.3f} ms/step, "
            f"{100 * b1_frac:.1f}% of HBM peak")
    except Exception as e:  # the headline number stands on its own
        log("[bench] batch-1 leg failed:", e)

    cpu, cpu_configs = (None, None) if args.no_cpu else cpu_baseline(B, pos0 + args.steps // 2)

    # prefill: all projections of every prompt token, causal attention, the LM head for the
    # last position of each sequence
    prefill_flops = (2.0 * B * P * L * (4 * d * d + 3 * d * F) + B * 4.0 * L * H * (P * P / 2.0) * dh
                     + 2.0 * B * V * d)
    lm.close()
    llama_bf16 = None
    if not args.no_bf16:
        try:
            llama_bf16 = run_llama_bf16(jas, args)
        except Exception as e:  # the headline number stands on its own
            log("[bench] bf16 leg failed:", e)
    gpt2 = tiny = None
    if not args.no_gpt2:
        try:
            g_tok, g_ms, g_bytes = run_gpt2(jas, (12, 768, 12, 3072, 50257, 1024), 8, 512, 3, 32, 4,
                                            graph=not args.no_graph)
            g_frac = g_bytes / (g_ms * 1e-3) / 1e9 / HBM_PEAK_GBS
            gpt2 = {"decode_tok_s": round(g_tok, 1), "ms_per_step": round(g_ms, 3),
                    "hbm_bytes_per_step": round(g_bytes), "step_hbm_frac": round(g_frac, 4),
                    "prefill": dict(run_gpt2.last_prefill, workload="8 x 512 prompt tokens, fp32, wall time"),
                    "workload": "config4: GPT-2-small fp32, batch 8, 512-token prompts, greedy decode "
                                "(32 timed steps after 4 warm-up)"}
            log(f"[bench] gpt2-small decode: {g_tok:.1f} tok/s, {g_ms:.3f} ms/step, {100 * g_frac:.1f}% of HBM peak; "
                f"prefill {run_gpt2.last_prefill}")
            t_tok, t_ms, t_bytes = run_gpt2(jas, (2, 128, 4, 512, 256, 64), 1, 32, 0, 31, 1,
                                            graph=not args.no_graph)
            tiny = {"decode_tok_s": round(t_tok, 1), "ms_per_step": round(t_ms, 4),
                    "workload": "config1: tiny GPT-2 fp32 (2 layers, d 128), batch 1, 32-token prompt, "
                                "32 greedy steps (31 timed after 1 warm-up)",
                    "bound": "launch latency (about 8 kernels per layer; %.2f MB of weights and KV per step)"
                             % (t_bytes / 1e6)}
            log(f"[bench] tiny gpt2 decode: {t_tok:.1f} tok/s, {1e3 * t_ms:.1f} us/step")
        except Exception as e:  # the headline number stands on its own
            log("[bench] gpt2 legs failed:", e)

    encdec = None
    if not args.no_encdec:
        try:
            encdec = run_encdec()
        except Exception as e:  # the headline number stands on its own
            log("[bench] encoder-decoder leg failed:", e)

    line = {
        "metric": "decode tok/s (GPT-2-small, LLaMA-7B shape); kernel % of HBM/MFMA peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * dt / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random-init N(0,0.02) weights, uniform random prompt ids)",
        "config": {"workload": f"config5: LLaMA-7B-shape decoder fp32, batch {B}, {P}-token prompts, "
                               f"greedy KV-cache decode (timed positions {pos0}..{pos0 + args.steps - 1})",
                   "batch": B, "prompt": P, "parallelism": "single GPU"},
        "roofline": roof,
        "roofline_other": {"kernel": other["kernel"], "achieved": round(other["achieved"], 1), "unit": "GB/s",
                           "frac": round(other["achieved"] / HBM_PEAK_GBS, 4)},
        "step_hbm_frac": round(step_roofline_frac, 4),
        "step_bytes": step_bytes_timed,
        "profiled_pass": {"steps": args.steps, "positions": [pos1, pos1 + args.steps - 1],
                          "gpu_ms_by_class": {"weight_gemm": round(ms[0], 3), "attention": round(ms[1], 3),
                                              "other": round(ms[2], 3)},
                          "launches_by_class": {"weight_gemm": cnt[0], "attention": cnt[1], "other": cnt[2]},
                          "wall_s": round(dt_prof, 4)},
        "prefill_tok_s": round(B * P / prefill_s, 1),
        "prefill_mfma": {"tflops": round(prefill_flops / prefill_s / 1e12, 2), "peak": 157.3,
                         "frac": round(prefill_flops / prefill_s / 1e12 / 157.3, 4),
                         "flops": prefill_flops, "note": "fp32 MFMA peak; wall time of the whole prefill"},
        "cpu_baseline": cpu,
        "cpu_configs": cpu_configs,
        "llama7b_batch1": b1,
        "llama7b_bf16_storage": llama_bf16,
        "gpt2_small": gpt2,
        "tiny_gpt2": tiny,
        "encdec_cpp_api": encdec,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
