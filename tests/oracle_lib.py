"""ctypes bindings to the test oracles (TEST INFRASTRUCTURE ONLY).

* ``orc``  -- oracle/liboracle.so, the C restatement of jasmine's arithmetic.
* ``ref``  -- oracle/_ref/libjasref.so, the jasmine reference compiled from its own
  headers (present only where it was built; ``None`` otherwise).
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# JAS_ORACLE_SO selects another build of the restatement (the sanitizer build, oracle/_san)
ORACLE_SO = os.environ.get("JAS_ORACLE_SO") or os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libjasref.so")

FP = C.POINTER(C.c_float)
IP = C.POINTER(C.c_int32)


def fp(a):
    return a.ctypes.data_as(FP) if a is not None else None


def ip(a):
    return a.ctypes.data_as(IP) if a is not None else None


def _load(path):
    if not os.path.exists(path):
        return None
    return C.CDLL(path)


orc = _load(ORACLE_SO)
ref = _load(REF_SO)

if orc is not None:
    orc.orc_normal.restype = C.c_float
    orc.orc_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_float]
    orc.orc_fill_normal.argtypes = [FP, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float, C.c_float]
    orc.orc_fill_randint.argtypes = [IP, C.c_size_t, C.c_uint64, C.c_uint64, C.c_uint32]
    orc.orc_gemm.argtypes = [C.c_int, C.c_int, C.c_int, FP, C.c_long, C.c_long, FP, C.c_long, C.c_long, FP, C.c_long]
    orc.orc_cfg2_expr.argtypes = [FP, FP, FP, FP, C.c_size_t]
    for n in ("orc_hsoftmax", "orc_softmax_global"):
        getattr(orc, n).argtypes = [FP, C.c_int, C.c_int, FP]
    for n in ("orc_hsum", "orc_vsum", "orc_hmax", "orc_vmean", "orc_hmean"):
        getattr(orc, n).argtypes = [FP, C.c_int, C.c_int, FP]
    orc.orc_sum.restype = C.c_float
    orc.orc_sum.argtypes = [FP, C.c_int, C.c_int]
    orc.orc_max.restype = C.c_float
    orc.orc_max.argtypes = [FP, C.c_int, C.c_int]
    orc.orc_linear.argtypes = [FP, FP, FP, C.c_int, C.c_int, C.c_int, FP]
    orc.orc_relu.argtypes = [FP, C.c_size_t, FP]
    orc.orc_sigmoid.argtypes = [FP, C.c_size_t, FP]
    orc.orc_layernorm_cols_jas.argtypes = [FP, C.c_int, C.c_int, FP, FP, FP]
    orc.orc_layernorm_rows.argtypes = [FP, C.c_int, C.c_int, C.c_float, FP, FP, FP]
    orc.orc_rmsnorm_rows.argtypes = [FP, C.c_int, C.c_int, C.c_float, FP, FP]
    orc.orc_gelu.restype = C.c_float
    orc.orc_gelu.argtypes = [C.c_float]
    orc.orc_silu.restype = C.c_float
    orc.orc_silu.argtypes = [C.c_float]
    orc.orc_jas_head.argtypes = [FP, FP, C.c_int, C.c_int, C.c_int, FP, FP, FP, FP, FP, FP, C.c_int, FP]
    orc.orc_jas_mha_nparams.restype = C.c_size_t
    orc.orc_jas_mha_nparams.argtypes = [C.c_int, C.c_int]
    orc.orc_jas_mha.argtypes = [FP, FP, C.c_int, C.c_int, C.c_int, C.c_int, FP, C.c_int, FP]
    orc.orc_attention.argtypes = [FP, FP, FP, FP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_double, C.c_int]
    orc.orc_rope_jas.argtypes = [FP, C.c_int, C.c_int, FP]
    orc.orc_rope_llama.argtypes = [FP, C.c_int, C.c_int, C.c_float]
    orc.orc_jas_encoder_layer_nparams.restype = C.c_size_t
    orc.orc_jas_encoder_layer_nparams.argtypes = [C.c_int, C.c_int]
    orc.orc_jas_decoder_layer_nparams.restype = C.c_size_t
    orc.orc_jas_decoder_layer_nparams.argtypes = [C.c_int, C.c_int]
    orc.orc_jas_transformer.argtypes = [FP, C.c_int, FP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, FP, FP]
    orc.orc_argmax.restype = C.c_int
    orc.orc_argmax.argtypes = [FP, C.c_int]


class LmCfg(C.Structure):
    _fields_ = [("kind", C.c_int), ("n_layer", C.c_int), ("d_model", C.c_int), ("n_head", C.c_int),
                ("d_ff", C.c_int), ("vocab", C.c_int), ("max_ctx", C.c_int),
                ("eps", C.c_float), ("rope_theta", C.c_float), ("kv_bf16", C.c_int)]


LM_WEIGHT_FIELDS = ["wte", "wpe", "ln1_g", "ln1_b", "w_qkv", "b_qkv", "w_o", "b_o", "ln2_g", "ln2_b",
                    "w_fc", "b_fc", "w_proj", "b_proj", "w_gate", "w_up", "w_down",
                    "lnf_g", "lnf_b", "w_head"]


class LmWeights(C.Structure):
    _fields_ = [(n, FP) for n in LM_WEIGHT_FIELDS]


if orc is not None:
    orc.orc_lm_generate.argtypes = [C.POINTER(LmCfg), C.POINTER(LmWeights), C.c_int, C.c_int, IP, C.c_int,
                                    IP, IP, FP, C.c_int]
    orc.orc_lm_last_logits.argtypes = [C.POINTER(LmCfg), C.POINTER(LmWeights), C.c_int, C.c_int, IP, FP, C.c_int]

if ref is not None:
    ref.ref_gemm.argtypes = [C.c_int, C.c_int, C.c_int, FP, FP, FP]
    ref.ref_gemm_tn.argtypes = [C.c_int, C.c_int, C.c_int, FP, FP, FP]
    ref.ref_cfg2_expr.argtypes = [FP, FP, FP, FP, C.c_int, C.c_int]
    ref.ref_expr.argtypes = [C.c_int, FP, C.c_int, C.c_int, FP, C.c_int, C.c_int, FP, IP, IP]
    ref.ref_hsoftmax.argtypes = [FP, C.c_int, C.c_int, FP]
    ref.ref_softmax_global.argtypes = [FP, C.c_int, C.c_int, FP]
    ref.ref_reductions.argtypes = [FP, C.c_int, C.c_int, FP, FP, FP, FP, FP, FP]
    ref.ref_linear.argtypes = [FP, FP, FP, C.c_int, C.c_int, C.c_int, FP]
    ref.ref_relu.argtypes = [FP, C.c_int, C.c_int, FP]
    ref.ref_sigmoid.argtypes = [FP, C.c_int, C.c_int, FP]
    ref.ref_layernorm_cols.argtypes = [FP, C.c_int, C.c_int, FP]
    ref.ref_head.argtypes = [FP, FP, C.c_int, C.c_int, C.c_int, FP, C.c_int, FP]
    ref.ref_mha.argtypes = [FP, FP, C.c_int, C.c_int, C.c_int, C.c_int, FP, C.c_int, FP]
    ref.ref_rope.argtypes = [FP, C.c_int, C.c_int, FP]
    ref.ref_transformer.argtypes = [FP, C.c_int, FP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, FP, FP]
    ref.ref_predict_loop.argtypes = [FP, C.c_int, FP, C.c_int, C.c_int, C.c_int, C.c_int, FP, C.c_int, FP]
    ref.ref_transformer_nparams.restype = C.c_long
    ref.ref_transformer_nparams.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int]
    for n, k in (("ref_time_linear", 4), ("ref_time_cfg2", 3), ("ref_time_hsoftmax", 3), ("ref_time_head", 3),
                 ("ref_time_attention_head", 2)):
        getattr(ref, n).restype = C.c_double
        getattr(ref, n).argtypes = [C.c_int] * k
    for n in ("ref_time_llama_layer", "ref_time_gpt2_layer"):
        getattr(ref, n).restype = C.c_double
        getattr(ref, n).argtypes = [C.c_int] * 4 + [C.POINTER(C.c_double)]
    ref.ref_time_prefill_layer.restype = C.c_double
    ref.ref_time_prefill_layer.argtypes = [C.c_int] * 5 + [C.POINTER(C.c_double)]


def normal(shape, seed, stream=0, mean=0.0, std=1.0):
    """Seeded N(mean, std) float32 array from the shared counter-based generator."""
    a = np.empty(int(np.prod(shape)), np.float32)
    orc.orc_fill_normal(fp(a), a.size, seed, stream, mean, std)
    return a.reshape(shape)


def randint(shape, n, seed, stream=0):
    a = np.empty(int(np.prod(shape)), np.int32)
    orc.orc_fill_randint(ip(a), a.size, seed, stream, n)
    return a.reshape(shape)
