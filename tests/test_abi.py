"""libheatkv.so loads on the host and exports every entry point of include/heatkv.h.

No kernel is launched here (there is no GPU on the build host); only the
loader functions and the argument checks that fail before any device call.
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from heatkv_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "heatkv.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:[\w\s\*]+?)\b(hkv_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_entry_points():
    names = _declared()
    for n in ("hkv_version", "hkv_device_ok", "hkv_last_error", "hkv_pack_segments",
              "hkv_segmented_attention", "hkv_segmented_attention_workspace_bytes"):
        assert n in names
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libheatkv.so not built")
    lib = _lib.load()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True)
    exported = set(re.findall(r"\sT\s(\w+)$", out.stdout, flags=re.M))
    for name in _declared():
        assert name in exported, name
        assert getattr(lib, name) is not None


def test_version_and_host_only_calls():
    lib = _lib.load()
    assert lib.hkv_version() == 0x000300 == _lib.ABI_VERSION
    assert lib.hkv_device_ok(-1) == 0
    assert isinstance(_lib.last_error(), str)


def test_header_and_integration_stub_carry_the_bindings_version():
    """HKV_VERSION in the header and the version the integration guide's
    ctypes stub checks are the one the bindings expect."""
    m = re.search(r"#define\s+HKV_VERSION\s+\(\((\d+) << 16\) \| \((\d+) << 8\) \| (\d+)\)", open(HEADER).read())
    assert m and (int(m.group(1)) << 16 | int(m.group(2)) << 8 | int(m.group(3))) == _lib.ABI_VERSION
    guide = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    checks = re.findall(r"hkv_version\(\)\s*==\s*(0x[0-9a-fA-F]+)", guide)
    assert checks and all(int(c, 16) == _lib.ABI_VERSION for c in checks)


def test_argument_errors_before_any_device_call():
    lib = _lib.load()
    null = None
    # head_dim 64 -> unsupported (RuntimeError in Python)
    code = lib.hkv_segmented_attention(null, null, null, null, null, null, null, null, null, null,
                                       1, 1, 1, 0, 0, 64, 2, 2, 2, 0, ctypes.c_float(1.0), 0, 0, 0, null, 0, null, 0, null)
    assert code == _lib.HKV_ERR_UNSUPPORTED and "head_dim=128" in _lib.last_error()
    with pytest.raises(RuntimeError, match="head_dim=128"):
        _lib.check(code)
    # q/k dtype mismatch
    code = lib.hkv_segmented_attention(null, null, null, null, null, null, null, null, null, null,
                                       1, 1, 1, 0, 0, 128, 3, 2, 2, 0, ctypes.c_float(1.0), 0, 0, 0, null, 0, null, 0, null)
    assert code == _lib.HKV_ERR_UNSUPPORTED
    # null pointers -> invalid argument (ValueError)
    code = lib.hkv_segmented_attention(null, null, null, null, null, null, null, null, null, null,
                                       1, 1, 1, 0, 0, 128, 2, 2, 2, 0, ctypes.c_float(1.0), 0, 0, 0, null, 0, null, 0, null)
    assert code == _lib.HKV_ERR_INVALID_ARG
    with pytest.raises(ValueError):
        _lib.check(code)
    # too many segments
    code = lib.hkv_segmented_attention(null, null, null, null, null, null, null, null, null, null,
                                       1, 1, 1, 10, 300, 128, 2, 2, 2, 0, ctypes.c_float(1.0), 0, 0, 0, null, 0, null, 0, null)
    assert code == _lib.HKV_ERR_UNSUPPORTED and "max_segments" in _lib.last_error()
    # pack: empty work is a no-op success, bad head_dim / element size rejected
    assert lib.hkv_pack_segments(null, null, null, null, 0, 0, 0, 0, 1, 128, 2, 2, null, null, null,
                                 0, 10, null) == 0
    assert lib.hkv_pack_segments(null, null, null, null, 0, 0, 0, 0, 1, 256, 2, 2, null, null, null,
                                 3, 10, null) == _lib.HKV_ERR_UNSUPPORTED
    assert lib.hkv_pack_segments(null, null, null, null, 0, 0, 0, 0, 1, 128, 8, 2, null, null, null,
                                 3, 10, null) == _lib.HKV_ERR_UNSUPPORTED
    assert lib.hkv_pack_segments(null, null, null, null, 0, 0, 0, 0, 1, 128, 2, 2, null, null, null,
                                 3, 10, null) == _lib.HKV_ERR_INVALID_ARG
    # bad output dtype
    code = lib.hkv_segmented_attention(null, null, null, null, null, null, null, null, null, null,
                                       1, 1, 1, 0, 0, 128, 2, 2, 2, 7, ctypes.c_float(1.0), 0, 0, 0, null, 0, null, 0, null)
    assert code == _lib.HKV_ERR_UNSUPPORTED and "out_dtype" in _lib.last_error()
    # dot modes outside the reference's ids
    for qk, vm in ((3, 0), (-1, 0), (0, 1), (0, 3)):
        code = lib.hkv_segmented_attention(null, null, null, null, null, null, null, null, null, null,
                                           1, 1, 1, 0, 0, 128, 2, 2, 2, 0, ctypes.c_float(1.0), 0, qk, vm,
                                           null, 0, null, 0, null)
        assert code == _lib.HKV_ERR_INVALID_ARG and "dot_mode" in _lib.last_error()
    # without a device the workspace size cannot be queried
    if not torch.cuda.is_available():
        assert lib.hkv_segmented_attention_workspace_bytes(0) == _lib.HKV_ERR_DEVICE


def test_qkv_produce_argument_errors():
    lib = _lib.load()
    null = None
    eps = ctypes.c_float(1e-12)

    def call(**kw):
        a = dict(qkv=null, stride=3 * 16 * 128, rope=null, rows=0, start=0, append=null, cap=0,
                 B=1, H=16, L=4, Dh=128, dt_in=2, dt_q=3, dt_k=3, dt_v=2, eps=eps)
        a.update(kw)
        return lib.hkv_qkv_produce(a["qkv"], a["stride"], null, null, null, a["rope"], a["rows"], a["start"],
                                   null, null, null, null, null, a["append"], a["cap"], a["B"], a["H"], a["L"],
                                   a["Dh"], a["dt_in"], a["dt_q"], a["dt_k"], a["dt_v"], 1, a["eps"], null)

    assert call(Dh=64) == _lib.HKV_ERR_UNSUPPORTED and "head_dim=128" in _lib.last_error()
    assert call(dt_in=3) == _lib.HKV_ERR_UNSUPPORTED
    assert call(dt_q=1) == _lib.HKV_ERR_UNSUPPORTED
    assert call(L=0) == _lib.HKV_OK  # empty scale: nothing to do
    assert call(H=0) == _lib.HKV_ERR_INVALID_ARG
    assert call(stride=100) == _lib.HKV_ERR_INVALID_ARG and "token_stride" in _lib.last_error()
    assert call() == _lib.HKV_ERR_INVALID_ARG and "null" in _lib.last_error()
    assert call(eps=ctypes.c_float(-1.0)) == _lib.HKV_ERR_INVALID_ARG


def test_bind_refuses_small_or_unbound_blocks():
    """The bound-call entry points reject a block that is too small and a
    block that was never bound, before touching any device."""
    lib = _lib.load()
    size = int(lib.hkv_segmented_attention_bound_bytes())
    assert 64 <= size <= 4096
    small = (ctypes.c_int64 * 1)()
    code = lib.hkv_segmented_attention_bind(ctypes.addressof(small), 8, None, None, None, 1, 1, 1, 0, 0, 128,
                                            2, 2, 2, 0, 1.0, 0, 0, 0, None, 0, None, 0, None)
    assert code == _lib.HKV_ERR_INVALID_ARG
    blank = (ctypes.c_int64 * ((size + 7) // 8))()
    code = lib.hkv_segmented_attention_call(ctypes.addressof(blank), 1, 1, 1, 1, 1, 1, None)
    assert code == _lib.HKV_ERR_INVALID_ARG
