"""ctypes binding of libheatkv.so (C ABI in include/heatkv.h).

The library is built in-tree (``heatkv_amd/libheatkv.so``) by
``heatkv_amd.csrc.build``.  There is no fallback: every entry point raises
``RuntimeError`` when the library is missing or the device is not a gfx950.
torch is imported before the library is opened so that the library binds to
the HIP runtime torch already loaded (both share the soname libamdhip64.so.7).
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libheatkv.so")

HKV_OK = 0
HKV_ERR_INVALID_ARG = -1
HKV_ERR_UNSUPPORTED = -2
HKV_ERR_LAUNCH = -3
HKV_ERR_DEVICE = -4

# HKV_VERSION of include/heatkv.h these bindings follow (SIGNATURES below);
# load() refuses a library built from another version of the header.
ABI_VERSION = (0 << 16) | (3 << 8) | 0

DTYPE_CODES = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3}
DTYPE_SPLIT_ROWS = 4  # K only: fp32 rows as bf16 high parts then low parts (hkv_split_rows)

# Leading bytes of the attention workspace that must be zero before a call
# (the per-item counters; the partial records behind them are written before
# they are read).
WORKSPACE_COUNTER_BYTES = 64 * 1024

_lock = threading.Lock()
_lib = None
_device_ok: dict[int, bool] = {}

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/heatkv.h
SIGNATURES = {
    "hkv_version": (_c_i32, []),
    "hkv_device_ok": (_c_i32, [_c_i32]),
    "hkv_last_error": (ctypes.c_char_p, []),
    "hkv_pack_segments": (
        _c_i32,
        [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
         _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_p],
    ),
    "hkv_segmented_attention": (
        _c_i32,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32,
         _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, ctypes.c_float, _c_i32, _c_i32,
         _c_i32, _c_p, _c_i32, _c_p, _c_i64, _c_p],
    ),
    "hkv_segmented_attention_append": (
        _c_i32,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32,
         _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, ctypes.c_float, _c_i32, _c_i32,
         _c_i32, _c_p, _c_i32, _c_p, _c_i64, _c_p, _c_p],
    ),
    "hkv_segmented_attention_append2": (
        _c_i32,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32,
         _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, ctypes.c_float, _c_i32, _c_i32,
         _c_i32, _c_p, _c_i32, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p],
    ),
    "hkv_segmented_attention_noalloc": (
        _c_i32,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32,
         _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, ctypes.c_float, _c_i32, _c_i32,
         _c_i32, _c_p, _c_i32, _c_p],
    ),
    "hkv_segmented_attention_bound_bytes": (_c_i64, []),
    "hkv_segmented_attention_bind": (
        _c_i32,
        [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
         _c_i32, ctypes.c_float, _c_i32, _c_i32, _c_i32, _c_p, _c_i32, _c_p, _c_i64, _c_p],
    ),
    "hkv_segmented_attention_bind2": (
        _c_i32,
        [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
         _c_i32, ctypes.c_float, _c_i32, _c_i32, _c_i32, _c_p, _c_i32, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64,
         _c_p],
    ),
    "hkv_segmented_attention_call": (_c_i32, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "hkv_segmented_attention_plan": (
        _c_i32, [_c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_i32]),
    "hkv_segmented_attention_item_shape": (_c_i32, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p]),
    "hkv_split_rows": (_c_i32, [_c_p, _c_p, _c_i64, _c_p]),
    "hkv_concat_kv": (_c_i32, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p]),
    "hkv_segmented_attention_slots": (_c_i32, [_c_i32]),
    "hkv_segmented_attention_workspace_bytes": (_c_i64, [_c_i32]),
    "hkv_qkv_produce": (
        _c_i32,
        [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
         _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
         ctypes.c_float, _c_p],
    ),
}


def load():
    """Open libheatkv.so once and return the ctypes handle (RuntimeError if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libheatkv.so not found at {LIB_PATH}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` or "
                "`python heatkv_amd/csrc/build.py`"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        have = int(lib.hkv_version())
        if have != ABI_VERSION:
            raise RuntimeError(
                f"{LIB_PATH} reports ABI version {have >> 16}.{(have >> 8) & 255}.{have & 255}; these "
                f"bindings need {ABI_VERSION >> 16}.{(ABI_VERSION >> 8) & 255}.{ABI_VERSION & 255} -- rebuild it "
                "with `python heatkv_amd/csrc/build.py`")
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().hkv_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(code: int) -> None:
    """Map a negative HKV_ERR_* code to ValueError / RuntimeError."""
    if code == HKV_OK:
        return
    msg = last_error() or f"libheatkv error {code}"
    if code == HKV_ERR_INVALID_ARG:
        raise ValueError(msg)
    raise RuntimeError(msg)


def require_device(device: torch.device) -> None:
    """RuntimeError unless ``device`` is a gfx950 GPU the library can run on."""
    lib = load()
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ok = _device_ok.get(idx)
    if ok is None:
        ok = bool(lib.hkv_device_ok(idx))
        _device_ok[idx] = ok
    if not ok:
        name = torch.cuda.get_device_name(idx) if torch.cuda.is_available() else "none"
        raise RuntimeError(f"libheatkv.so runs on gfx950 (MI355X) only; device {idx} is {name}")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    return DTYPE_CODES.get(dtype, 0)


# Attention workspaces, one per (device, stream): calls on one stream run in
# order, so they can share one; calls on different streams may overlap.
_workspaces: dict = {}
# Under HIP-graph capture: one per (device, stream) and capture, from the
# graph's own pool: (capture id, tensor).
_capture_workspaces: dict = {}
_hip_rt = None


def _hip_runtime():
    """The HIP runtime library torch loaded (for stream-capture queries)."""
    global _hip_rt
    if _hip_rt is None:
        path = "libamdhip64.so"
        try:
            with open("/proc/self/maps") as fh:
                for line in fh:
                    if "libamdhip64" in line:
                        path = line.split()[-1]
                        break
        except OSError:
            pass
        lib = ctypes.CDLL(path)
        fn = lib.hipStreamGetCaptureInfo
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_ulonglong)]
        _hip_rt = lib
    return _hip_rt


def capture_id(stream_handle: int) -> int:
    """Id of the graph capture running on the stream (0 when none)."""
    status = ctypes.c_int(0)
    cid = ctypes.c_ulonglong(0)
    err = _hip_runtime().hipStreamGetCaptureInfo(ctypes.c_void_p(stream_handle), ctypes.byref(status),
                                                 ctypes.byref(cid))
    if err != 0:
        raise RuntimeError(f"hipStreamGetCaptureInfo failed with HIP error {err}")
    return int(cid.value) if status.value == 1 else 0  # 1 = hipStreamCaptureStatusActive


# os.environ keeps its values in a dict of encoded keys (CPython on POSIX;
# os.environ[...] = ... and del os.environ[...] update it): a knob read from
# that dict costs ~0.1 us, through os.environ.get ~0.8 us, and an operator
# call reads about ten knobs.
_ENV_DATA = getattr(os.environ, "_data", None)
_ENV_KEYS: dict = {}


def env_get(name: str, default=None):
    """``os.environ.get(name, default)``, read from the environment's own dict."""
    if isinstance(_ENV_DATA, dict):
        key = _ENV_KEYS.get(name)
        if key is None:
            try:
                key = _ENV_KEYS[name] = os.environ.encodekey(name)
            except Exception:  # pragma: no cover - another platform's os.environ
                return os.environ.get(name, default)
        raw = _ENV_DATA.get(key)
        return default if raw is None else os.environ.decodevalue(raw)
    return os.environ.get(name, default)


def attention_workspace(device: torch.device, stream=None):
    """Workspace tensor (counters zeroed) of ``hkv_segmented_attention`` for the
    current stream of ``device`` (or ``stream``, that stream) -- None when
    HKV_ATTN_SPLIT=0: no item is cut.  The kernels leave the counters zeroed,
    so a stream's workspace is allocated and cleared once; under HIP-graph
    capture, once per capture (from the graph's pool, cleared by a fill kernel
    that the graph replays before the first call, no memset node)."""
    if env_get("HKV_ATTN_SPLIT", "1") == "0":
        return None
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if stream is None:
        stream = torch.cuda.current_stream(idx)
    key = (idx, stream.cuda_stream)
    if torch.cuda.is_current_stream_capturing():
        cid = capture_id(stream.cuda_stream)
        hit = _capture_workspaces.get(key)
        if hit is not None and hit[0] == cid:
            return hit[1]
        need = int(load().hkv_segmented_attention_workspace_bytes(idx))
        if need < 0:
            check(need)
        ws = torch.empty(need, dtype=torch.uint8, device=torch.device("cuda", idx))
        ws[:WORKSPACE_COUNTER_BYTES].zero_()
        _capture_workspaces[key] = (cid, ws)  # an earlier capture's buffer stays with its graph
        return ws
    ws = _workspaces.get(key)
    if ws is None:
        need = int(load().hkv_segmented_attention_workspace_bytes(idx))
        if need < 0:
            check(need)
        ws = torch.zeros(need, dtype=torch.uint8, device=torch.device("cuda", idx))
        _workspaces[key] = ws
    return ws
