"""jasmine_amd -- MI355X (gfx950) implementation of jasmine's transformer inference path.

The product is libjasmine_hip.so (C ABI declared in include/jasmine_hip.h) plus the
C++20 headers under jasmine_amd/include that keep jasmine's mat_t / mat_express_t /
mat_net_t / mat_mha_t / mat_transformer_t API.  This module is a thin ctypes binding of
the C ABI used by the tests and bench.py.  There is no CPU fallback: importing the
binding without the built library raises.
"""
from .capi import lib, LIB_PATH, JasError, check, DeviceArray, to_device, LmConfig, Lm, leaf, read_lm_config  # noqa: F401

__all__ = ["lib", "LIB_PATH", "JasError", "check", "DeviceArray", "to_device", "LmConfig", "Lm", "leaf", "read_lm_config"]
