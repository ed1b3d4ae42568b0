"""Weight files of the LM runner (jas_lm_save / jas_lm_load / jas_lm_read_config).

The container is safetensors; these tests write and read it with the `safetensors` Python
package (an independent implementation of the format), so the library's reader and writer
are checked against a third party, not against each other.  The reference has no weight
file (its nets take weights through init_weight<I>(), mat_init_t.hpp:113-118), so there is
no reference fixture to match: parity here is bit-exact equality of the weights and of the
generated ids / logits across a save -> load round trip.

CPU tests parse headers only (jas_lm_read_config makes no device call); GPU tests move
weights through the device.
"""
import json
import os
import struct

import numpy as np
import pytest

from oracle_lib import randint

CFG_KEYS = ("kind", "n_layer", "d_model", "n_head", "d_ff", "vocab", "max_ctx", "max_batch", "eps",
            "rope_theta", "weight_bf16", "kv_bf16")


def capi():
    import jasmine_amd.capi as c
    return c


def write_raw(path, header, data=b"", pad=True):
    """A safetensors file from an explicit header object (or text) and data bytes."""
    h = header if isinstance(header, (bytes, str)) else json.dumps(header)
    h = h.encode() if isinstance(h, str) else h
    if pad:
        h += b" " * ((8 - (8 + len(h)) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)


def meta_for(cfg_vals):
    m = {"format": "jasmine_amd.lm"}
    m.update({k: str(v) for k, v in zip(CFG_KEYS, cfg_vals)})
    return m


# ------------------------------------------------------------------ CPU: header and config
def test_read_config_from_safetensors_package(tmp_path):
    from safetensors.numpy import save_file
    c = capi()
    vals = (1, 3, 256, 2, 512, 320, 48, 3, 1e-6, 10000.0, 1, 0)
    p = str(tmp_path / "w.safetensors")
    save_file({"lnf_g": np.ones((1, 1, 256), np.float32)}, p, metadata=meta_for(vals))
    cfg = c.read_lm_config(p)
    got = tuple(getattr(cfg, k) for k in CFG_KEYS)
    assert got[:8] == vals[:8] and got[10:] == vals[10:]
    assert got[8] == np.float32(1e-6) and got[9] == 10000.0


def test_read_config_json_escapes(tmp_path):
    # escapes, a surrogate pair and non-ASCII names elsewhere in the header must parse
    c = capi()
    vals = (0, 2, 128, 4, 512, 256, 64, 1, 1e-5, 10000.0, 0, 0)
    hdr = ('{"caf\\u00e9 \\ud83d\\ude00 \\"q\\" \\\\ \\/ \\n": {"dtype": "F32", "shape": [2], '
           '"data_offsets": [0, 8]}, "__metadata__": ' + json.dumps(meta_for(vals)) + "}")
    p = str(tmp_path / "e.safetensors")
    write_raw(p, hdr, b"\0" * 8)
    cfg = c.read_lm_config(p)
    assert (cfg.kind, cfg.n_layer, cfg.vocab, cfg.max_ctx) == (0, 2, 256, 64)


@pytest.mark.parametrize("case", ["missing", "short", "badlen", "json", "trailing", "dtype", "offsets", "past_end",
                                  "shape", "nometa", "wrongformat", "badint", "lacks_key", "dup", "overflow"])
def test_header_errors(tmp_path, case):
    c = capi()
    vals = (0, 2, 128, 4, 512, 256, 64, 1, 1e-5, 10000.0, 0, 0)
    good_t = {"dtype": "F32", "shape": [1, 2], "data_offsets": [0, 8]}
    meta = meta_for(vals)
    p = str(tmp_path / "x.safetensors")
    code = 1
    if case == "missing":
        p, code = str(tmp_path / "does_not_exist"), 2
    elif case == "short":
        open(p, "wb").write(b"\x01\x00")
    elif case == "badlen":
        open(p, "wb").write(struct.pack("<Q", 1 << 40) + b"{}")
    elif case == "json":
        write_raw(p, '{"a": {"dtype": "F32",', b"\0" * 8)
    elif case == "trailing":
        write_raw(p, '{"__metadata__": ' + json.dumps(meta) + '} x', b"")
    elif case == "dtype":
        write_raw(p, {"a": dict(good_t, dtype="F16"), "__metadata__": meta}, b"\0" * 8)
    elif case == "offsets":
        write_raw(p, {"a": dict(good_t, data_offsets=[0, 12]), "__metadata__": meta}, b"\0" * 12)
    elif case == "past_end":
        write_raw(p, {"a": good_t, "__metadata__": meta}, b"\0" * 4)
    elif case == "shape":
        write_raw(p, {"a": dict(good_t, shape=[1, 1, 1, 2]), "__metadata__": meta}, b"\0" * 8)
    elif case == "nometa":
        write_raw(p, {"a": good_t}, b"\0" * 8)
    elif case == "wrongformat":
        write_raw(p, {"a": good_t, "__metadata__": dict(meta, format="other")}, b"\0" * 8)
    elif case == "badint":
        write_raw(p, {"a": good_t, "__metadata__": dict(meta, n_layer="2x")}, b"\0" * 8)
    elif case == "lacks_key":
        m = dict(meta)
        del m["rope_theta"]
        write_raw(p, {"a": good_t, "__metadata__": m}, b"\0" * 8)
    elif case == "overflow":  # 4 * 2^31 * 2^31 * 2^2 wraps to 0 in 64 bits
        write_raw(p, {"a": dict(good_t, shape=[2147483647, 2147483647, 4], data_offsets=[0, 0]),
                      "__metadata__": meta}, b"")
    elif case == "dup":
        write_raw(p, '{"a": %s, "a": %s, "__metadata__": %s}' % (json.dumps(good_t), json.dumps(good_t),
                                                                  json.dumps(meta)), b"\0" * 8)
    with pytest.raises(c.JasError) as e:
        c.read_lm_config(p)
    assert e.value.code == code, str(e.value)


# ------------------------------------------------------------------ GPU: weights through the device
def bf16_round(a):
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16).astype(np.uint32).view(np.float32)


def names_of(lm):
    import jasmine_amd as jas
    out = []
    for n in ("wte", "wpe", "ln1_g", "ln1_b", "w_qkv", "b_qkv", "w_o", "b_o", "ln2_g", "ln2_b", "w_fc", "b_fc",
              "w_proj", "b_proj", "w_gate", "w_up", "w_down", "lnf_g", "lnf_b", "w_head"):
        if lm.weight_shape(n)[0]:
            out.append(n)
    return out


CONFIGS = {  # kind, layers, d, heads, ffn, vocab, ctx, batch, eps, theta, weight_bf16, kv_bf16
    "gpt2": (0, 2, 128, 4, 512, 256, 64, 2, 1e-5, 10000.0, 0, 0),
    "llama": (1, 2, 256, 2, 512, 320, 48, 2, 1e-6, 10000.0, 0, 0),
    "llama_bf16": (1, 2, 256, 2, 512, 320, 48, 2, 1e-6, 10000.0, 1, 1),
    "gpt2_bf16": (0, 2, 192, 3, 336, 77, 40, 2, 1e-5, 10000.0, 1, 0),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CONFIGS))
def test_save_matches_weights_and_reloads_exactly(jas, tmp_path, name):
    import torch
    from safetensors.torch import load_file
    from safetensors import safe_open
    cfg = jas.LmConfig(*CONFIGS[name])
    a = jas.Lm(cfg)
    a.init_random(11, 0.02)
    p = str(tmp_path / "m.safetensors")
    a.save(p)
    # the third-party reader sees every weight, bit-exact, with its shape and storage dtype
    t = load_file(p)
    assert sorted(t) == sorted(names_of(a))
    for n in names_of(a):
        l, r, c = a.weight_shape(n)
        assert tuple(t[n].shape) == (l, r, c), n
        packed = n.startswith("w_") or (n == "wte" and cfg.kind == 0)
        assert t[n].dtype == (torch.bfloat16 if (packed and cfg.weight_bf16) else torch.float32), n
        got = t[n].float().numpy().ravel()
        assert np.array_equal(got.view(np.uint32), a.weight(n).view(np.uint32)), n
    with safe_open(p, "pt") as f:
        meta = f.metadata()
    assert meta["format"] == "jasmine_amd.lm"
    rc = jas.read_lm_config(p)
    for k in CFG_KEYS:
        assert getattr(rc, k) == getattr(cfg, k), k
    # a second model loaded from the file generates the same ids and logits, bit for bit
    b = jas.Lm(cfg)
    b.init_random(12, 0.02)
    b.load(p)
    for n in names_of(a):
        assert np.array_equal(a.weight(n).view(np.uint32), b.weight(n).view(np.uint32)), n
    prompt = randint((2, 9), cfg.vocab, 5)
    na, la = a.prefill(prompt, want_logits=True)
    nb, lb = b.prefill(prompt, want_logits=True)
    assert np.array_equal(na, nb) and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert np.array_equal(a.generate(6, 2), b.generate(6, 2))


@pytest.mark.gpu
@pytest.mark.parametrize("name,file_bf16", [("llama", 0), ("llama", 1), ("llama_bf16", 0), ("llama_bf16", 1),
                                            ("gpt2", 1), ("gpt2_bf16", 0)])
def test_load_third_party_file(jas, tmp_path, name, file_bf16):
    """A file written by the safetensors package (F32 or BF16 data, 2-D for single-layer
    tensors): F32 into bf16 storage rounds to nearest even, BF16 widens exactly."""
    import torch
    from safetensors.torch import save_file
    cfg = jas.LmConfig(*CONFIGS[name])
    lm = jas.Lm(cfg)
    rng = np.random.default_rng(3)
    want, tensors = {}, {}
    for n in names_of(lm):
        l, r, c = lm.weight_shape(n)
        x = (rng.standard_normal((l, r, c)) * 0.05).astype(np.float32)
        tt = torch.from_numpy(x[0] if l == 1 else x)
        if file_bf16:
            tt = tt.to(torch.bfloat16)
            x = tt.float().numpy().reshape(l, r, c)
        tensors[n] = tt.contiguous()
        packed = n.startswith("w_") or (n == "wte" and cfg.kind == 0)
        want[n] = bf16_round(x) if (packed and cfg.weight_bf16) else x
    p = str(tmp_path / "tp.safetensors")
    save_file(tensors, p)
    lm.load(p)
    for n in want:
        assert np.array_equal(lm.weight(n).view(np.uint32), want[n].ravel().view(np.uint32)), n


@pytest.mark.gpu
def test_load_longer_position_table(jas, tmp_path):
    from safetensors.numpy import save_file
    cfg = jas.LmConfig(*CONFIGS["gpt2"])
    a = jas.Lm(cfg)
    a.init_random(21, 0.02)
    t = {n: a.weight(n).reshape(a.weight_shape(n)) for n in names_of(a)}
    extra = np.full((1, 16, cfg.d_model), 7.0, np.float32)
    t["wpe"] = np.concatenate([t["wpe"], extra], 1)  # 16 more positions than max_ctx
    p = str(tmp_path / "wpe.safetensors")
    save_file(t, p)
    b = jas.Lm(cfg)
    b.load(p)
    assert np.array_equal(b.weight("wpe"), a.weight("wpe"))


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["lacks", "extra", "shape", "short_wpe"])
def test_load_rejects_mismatched_file(jas, tmp_path, case):
    from safetensors.numpy import save_file
    cfg = jas.LmConfig(*CONFIGS["gpt2"])
    a = jas.Lm(cfg)
    a.init_random(31, 0.02)
    t = {n: a.weight(n).reshape(a.weight_shape(n)) for n in names_of(a)}
    if case == "lacks":
        del t["b_o"]
    elif case == "extra":
        t["w_gate"] = np.zeros((2, 512, 128), np.float32)
    elif case == "shape":
        t["w_qkv"] = np.zeros((2, 3 * 128, 64), np.float32)
    elif case == "short_wpe":
        t["wpe"] = t["wpe"][:, :10]
    p = str(tmp_path / "bad.safetensors")
    save_file(t, p)
    before = a.weight("w_o").copy()
    with pytest.raises(jas.JasError) as e:
        a.load(p)
    assert e.value.code == 1, str(e.value)
    # validation happens before any upload: the model is unchanged
    assert np.array_equal(a.weight("w_o"), before)


@pytest.mark.gpu
def test_save_is_atomic_on_bad_path(jas, tmp_path):
    cfg = jas.LmConfig(*CONFIGS["gpt2"])
    a = jas.Lm(cfg)
    a.init_random(41, 0.02)
    with pytest.raises(jas.JasError):
        a.save(str(tmp_path / "no_such_dir" / "m.safetensors"))
    assert not os.path.exists(tmp_path / "no_such_dir")


def test_header_parser_survives_corruption(tmp_path):
    """Seeded byte flips, insertions and truncations of a valid file: the header parser
    returns a status (success or an error code) for every one and never crashes."""
    from safetensors.numpy import save_file
    c = capi()
    vals = (1, 2, 64, 2, 128, 100, 32, 2, 1e-6, 10000.0, 0, 0)
    src = str(tmp_path / "ok.safetensors")
    save_file({"lnf_g": np.ones((1, 1, 64), np.float32), "w_head": np.zeros((1, 100, 64), np.float32)}, src,
              metadata=meta_for(vals))
    good = open(src, "rb").read()
    hlen = struct.unpack("<Q", good[:8])[0]
    rng = np.random.default_rng(7)
    p = str(tmp_path / "bad.safetensors")
    outcomes = {0: 0, 1: 0, 2: 0}
    for _ in range(400):
        b = bytearray(good)
        kind = rng.integers(4)
        if kind == 0:  # flip bytes in the header
            for _ in range(int(rng.integers(1, 6))):
                b[8 + int(rng.integers(hlen))] = int(rng.integers(256))
        elif kind == 1:  # truncate anywhere
            b = b[:int(rng.integers(len(b)))]
        elif kind == 2:  # corrupt the length field
            b[int(rng.integers(8))] = int(rng.integers(256))
        else:  # insert a structural character
            i = 8 + int(rng.integers(hlen))
            b = b[:i] + bytes([b'{}[]",:\\'[int(rng.integers(8))]]) + b[i:]
        open(p, "wb").write(bytes(b))
        try:
            c.read_lm_config(p)
            outcomes[0] += 1
        except c.JasError as e:
            assert e.code in (1, 2), str(e)
            outcomes[e.code] += 1
    assert outcomes[1] > 100
