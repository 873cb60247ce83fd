"""The C-ABI library loads, exports every entry point include/xdna_engine.h
declares, and follows the npu-capi error convention (NULL / -1 plus a
thread-local message) -- CPU only, no compute calls."""
import ctypes as C
import os
import re

import pytest

from conftest import ROOT, load_xe

HEADER = os.path.join(ROOT, "include", "xdna_engine.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xe_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("xe_device_open", "xe_register_weight", "xe_gemv", "xe_fused_norm_gemv",
                 "xe_gemv_i8act", "xe_attn_decode", "xe_decoder_step", "xe_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    xe = load_xe()
    L = xe.lib()
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing
    # and the mirror binds exactly the declared surface
    assert sorted(xe.EXPORTS) == declared()


def test_abi_version():
    xe = load_xe()
    assert xe.lib().xe_abi_version() == 1


def test_error_convention_without_gpu_work():
    xe = load_xe()
    L = xe.lib()
    assert L.xe_gemv(None, None, None, 0, 1, None) == -1
    assert "null" in xe.last_error()
    assert L.xe_attn_decode(None, None, None, None, None, 1, 1, 1, 64, 16, 1.0, None) == -1
    assert L.xe_decoder_step(None, None, None, 1, None, None) == -1
    assert xe.last_error() != ""
    assert L.xe_buf_alloc(None, 16) is None
    assert L.xe_weight_shape(None, None, None, None) == -1


def test_device_open_out_of_range_fails_cleanly():
    xe = load_xe()
    n = xe.device_count()
    assert n >= 0
    assert xe.lib().xe_device_open(n + 7) is None
    assert xe.last_error() != ""
