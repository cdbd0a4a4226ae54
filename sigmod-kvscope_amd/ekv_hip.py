"""ctypes binding of ``lib/libekv_hip.so``, the C ABI declared in ``include/ekv_hip.h``.

The binding is thin: every call takes device addresses (``int``), element strides, sizes and a
stream handle, and a non-zero status becomes an exception with the library's message:
``EKV_EINVAL`` and ``EKV_EUNSUPPORTED`` raise ``ValueError``, ``EKV_ELAUNCH`` raises
``RuntimeError``, as the reference raises them for misuse and for device failures.  There is no
fallback: without the built library every entry point raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("EKV_HIP_LIB") or os.path.join(HERE, "lib", "libekv_hip.so")

OK, EINVAL, ELAUNCH, EUNSUPPORTED = 0, -1, -2, -3
F32, F16, BF16, FP8_E4M3, F64 = 0, 1, 2, 3, 4
AGG_MEAN, AGG_MAX = 0, 1
AUDIT_SELF_CONTAINED, AUDIT_PLANNED = 1, 2
OBJ_SUM, OBJ_MAXMIN = 0, 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_sz = ctypes.c_size_t


class AuditLayer(ctypes.Structure):
    """``ekv_audit_layer_t``: one layer of a multi-layer audit launch."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("keys", ctypes.c_void_p),
        ("layer", ctypes.c_int32),
        ("group_first", ctypes.c_int32),
        ("q_head0", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("k_scale", ctypes.c_float),
        ("pad", ctypes.c_int32),
    ]


_SIGNATURES: dict[str, list] = {
    "ekv_last_error": [],
    "ekv_abi_version": [],
    "ekv_audit_tile_lse": [
        _p, _i32, _i64, _i64,  # q, q dtype, strides
        _p, _i32, _i64, _i64, _i64, _f32,  # keys, kv dtype, strides, k_scale
        _p, _i64, _p, _p, _p, _p,  # table, stride, lens, qrow, select, flag
        _p, _i64, _i64, _i64, _i32,  # lse, plane / layer / row strides, cells
        _p, _i32,  # cycles, cycles_rows
        _f32, _i32, _i32, _i32, _i32,  # scale, layer, group_first, groups, group_rows
        _i32, _i32, _i32, _i32, _i32, _i32,  # rows, width, block_size, tile_blocks, head_dim, chunk_tiles
        _p,  # stream
    ],
    "ekv_audit_plan_bytes": [_i32, _i32],
    "ekv_audit_plan": [
        _p, _i64, _p, _p, _p, _p,  # table, stride, lens, qrow, select, flag
        _i32, _i32, _i32, _i32,  # rows, width, block_size, tile_blocks
        _p, _sz, _i32, _i32,  # plan, plan bytes, plan rows, plan width
        _p,  # stream
    ],
    "ekv_audit_tile_lse_planned": [
        _p, _i32, _i64, _i64,  # q, q dtype, strides
        _p, _i32, _i64, _i64, _i64, _f32,  # keys, kv dtype, strides, k_scale
        _p, _i64, _p, _p, _p, _p,  # table, stride, lens, qrow, select, flag
        _p, _i64, _i64, _i64, _i32,  # lse, plane / layer / row strides, cells
        _p, _i32,  # cycles, cycles_rows
        _f32, _i32, _i32, _i32, _i32,  # scale, layer, group_first, groups, group_rows
        _i32, _i32, _i32, _i32, _i32,  # rows, width, block_size, tile_blocks, head_dim
        _p, _sz, _i32, _i32,  # plan, plan bytes, plan rows, plan width
        _p,  # stream
    ],
    "ekv_audit_shape": [_i32, _i32, _i32, _i32],
    "ekv_audit_tile_lse_layers": [
        ctypes.POINTER(AuditLayer), _i32, _i32,  # layers, count, queries by row
        _i32, _i64, _i64,  # q dtype, strides
        _i32, _i64, _i64, _i64,  # kv dtype, strides
        _p, _i64, _p, _p, _p, _p,  # table, stride, lens, qrow, select, flag
        _p, _i64, _i64, _i64, _i32,  # lse, plane / layer / row strides, cells
        _p, _i32,  # cycles, cycles_rows
        _i32, _i32,  # groups, group_rows
        _i32, _i32, _i32, _i32, _i32,  # rows, width, block_size, tile_blocks, head_dim
        _p, _sz, _i32, _i32,  # plan, plan bytes, plan rows, plan width
        _p,  # stream
    ],
    "ekv_audit_stage_queries": [
        _p, _i32, _i64, _i64,  # q, q dtype, strides
        _i32, _i32, _i32,  # head_first, heads, head_dim
        _p, _p, _p, _i32,  # qrow, select, flag, rows
        _p, _i64,  # staged, staged row stride
        _p,  # stream
    ],
    "ekv_tile_shares": [_p, _i64, _i64, _i64, _i32, _i32, _i32, _p, _p, _i32, _i32, _i32, _p, _i64, _p],
    "ekv_tile_shares_workspace": [_i32, _i32, _i32],
    "ekv_tile_shares_ws": [_p, _i64, _i64, _i64, _i32, _i32, _i32, _p, _p, _i32, _i32, _i32, _p, _i64, _p, _sz, _p],
    "ekv_tile_shares_noalloc": [_p, _i64, _i64, _i64, _i32, _i32, _i32, _p, _p, _i32, _i32, _i32, _p, _i64, _p],
    "ekv_tile_shares_status": [_p, ctypes.POINTER(_i32)],
    "ekv_tile_shares_reset": [_p, _sz, _p],
    "ekv_tile_shares_test_wait": [_i32, _i32],
    "ekv_normalize_tile_lse": [_p, _i64, _i64, _i32, _i32, _i32, _p, _i32, _i32, _i32, _p, _i64, _p],
    "ekv_rank_uniform": [
        _p, _i64, _p, _p, _p, _i64, _p, _i32, _p, _i64, _i32, _i32, _f64, _i64, _p, _i64, _p, _p,
    ],
    "ekv_rank_uniform_ws": [
        _p, _i64, _p, _p, _p, _i64, _p, _i32, _p, _i64, _i32, _i32, _f64, _i64, _p, _i64, _p, _p, _p,
    ],
    "ekv_rank_uniform64_workspace": [_i32],
    "ekv_rank_uniform64": [
        _p, _i64, _p, _p, _p, _i64, _p, _i32, _p, _i64, _i32, _i32, _f64, _i64, _p, _i64, _p, _p, _sz, _p,
    ],
    "ekv_rank_uniform_view": [
        _p, _i64, _p, _p, _p, _i32, _i32, _i32, _f64, _i64, _p, _i64, _p, _p, _i64, _p, _i32, _p, _i64, _p, _p, _p,
    ],
    "ekv_compact_view": [_p, _i64, _p, _p, _i64, _i32, _i32, _i32, _p, _i64, _p, _p],
    "ekv_build_view": [
        _p, _i64, _p, _p, _i64, _p, _i64, _p, _p, _i32, _i32, _i32, _i32, _p, _i64, _p, _p, _p,
    ],
    "ekv_rank_sum_workspace": [_i32],
    "ekv_rank_sum": [_p, _i64, _p, _p, _p, _i64, _i32, _i32, _i64, _p, _i64, _p, _p, _sz, _p],
    "ekv_rank_maxmin_workspace": [_i32, _i32],
    "ekv_rank_maxmin": [_p, _i64, _p, _p, _i64, _i32, _i32, _i64, _p, _i64, _p, _p, _sz, _p],
    "ekv_controller_keep_workspace": [_i32, _i32, _i32],
    "ekv_controller_keep": [
        _i32, _p, _i32, _i64,  # objective, shares, dtype, stride
        _p, _p, _p, _p, _i64, _p,  # lengths, evidence, audited, released, stride, weights
        _i32, _i32, _i32, _i32, _f64,  # rows, width, recent, cap, fraction
        _p, _i64, _p, _p, _sz, _p,  # keep, stride, summary, workspace, bytes, stream
    ],
    "ekv_compact_slots": [
        _p, _p, _i32, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _i64, _p, _p, _p, _i64, _p, _p, _i32, _p,
    ],
    "ekv_malloc": [ctypes.POINTER(ctypes.c_void_p), _sz],
    "ekv_free": [_p],
    "ekv_memset": [_p, ctypes.c_int, _sz],
    "ekv_memcpy_h2d": [_p, _p, _sz],
    "ekv_memcpy_d2h": [_p, _p, _sz],
    "ekv_ipc_handle": [_p, ctypes.POINTER(ctypes.c_ubyte)],
    "ekv_ipc_open": [ctypes.POINTER(ctypes.c_ubyte), ctypes.POINTER(ctypes.c_void_p)],
    "ekv_synchronize": [],
    "ekv_device_count": [ctypes.POINTER(ctypes.c_int)],
}

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The loaded library, with its signatures set.  Raises ``RuntimeError`` if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built: run `python sigmod-kvscope_amd/build.py` (or __graft_entry__.build())"
        )
    # One HIP runtime per process, and the same in every process: torch ships its own, and the
    # library binds to whichever copy is loaded first.  Loading torch's first means a serving process
    # (which imports torch before anything else) and a reader process agree, so the IPC handles one
    # exports open in the other (handles of different runtime versions do not).
    import torch  # noqa: F401

    lib = ctypes.CDLL(LIB_PATH)
    for name, args in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        if name == "ekv_last_error":
            fn.restype = ctypes.c_char_p
        elif name.endswith("_workspace") or name.endswith("_bytes"):
            fn.restype = ctypes.c_size_t
        else:
            fn.restype = ctypes.c_int
    _lib = lib
    return lib


def exported() -> list[str]:
    """The entry points the binding expects the library to export."""
    return list(_SIGNATURES)


def check(status: int, what: str) -> None:
    if status == OK:
        return
    message = (load().ekv_last_error() or b"").decode(errors="replace") or what
    if status in (EINVAL, EUNSUPPORTED):
        raise ValueError(message)
    raise RuntimeError(message)


def call(name: str, *args) -> None:
    """Call entry point ``name`` and raise on a non-zero status."""
    check(getattr(load(), name)(*args), name)


def stream_handle(stream=None) -> int:
    """The raw hipStream_t of ``stream``: a torch stream, a raw handle (int) as is, or by default
    torch's current stream on the current device."""
    if isinstance(stream, int):
        return stream
    import torch

    s = torch.cuda.current_stream() if stream is None else stream
    return int(s.cuda_stream)


def malloc(nbytes: int) -> int:
    ptr = ctypes.c_void_p()
    call("ekv_malloc", ctypes.byref(ptr), nbytes)
    if not ptr.value:
        raise RuntimeError(f"hipMalloc of {nbytes} bytes returned null")
    return int(ptr.value)


def memset(address: int, value: int, nbytes: int) -> None:
    call("ekv_memset", address, value, nbytes)


def h2d(address: int, data: bytes | memoryview, nbytes: int | None = None) -> None:
    buf = (ctypes.c_char * len(data)).from_buffer_copy(data)
    call("ekv_memcpy_h2d", address, ctypes.addressof(buf), len(data) if nbytes is None else nbytes)


def d2h(address: int, nbytes: int) -> bytes:
    out = (ctypes.c_char * nbytes)()
    call("ekv_memcpy_d2h", ctypes.addressof(out), address, nbytes)
    return bytes(out)


def ipc_handle(address: int) -> bytes:
    handle = (ctypes.c_ubyte * 64)()
    call("ekv_ipc_handle", address, handle)
    return bytes(handle)


def ipc_open(handle: bytes) -> int:
    if len(handle) != 64:
        raise ValueError(f"an IPC handle has 64 bytes, got {len(handle)}")
    raw = (ctypes.c_ubyte * 64).from_buffer_copy(handle)
    ptr = ctypes.c_void_p()
    call("ekv_ipc_open", raw, ctypes.byref(ptr))
    if not ptr.value:
        raise RuntimeError("hipIpcOpenMemHandle returned a null pointer")
    return int(ptr.value)


def synchronize() -> None:
    call("ekv_synchronize")


def dtype_code(dtype) -> int:
    """The EKV_* element-type code of a torch dtype."""
    import torch

    codes = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
    fp8 = getattr(torch, "float8_e4m3fn", None)
    if fp8 is not None:
        codes[fp8] = FP8_E4M3
    if dtype not in codes:
        raise ValueError(f"unsupported element type {dtype}")
    return codes[dtype]


def ptr(tensor) -> int:
    """The device address of a torch tensor, or 0 for None."""
    return 0 if tensor is None else int(tensor.data_ptr())
