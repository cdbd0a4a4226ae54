"""The C ABI: the built library loads and exports every entry point include/ekv_hip.h declares, and the
ctypes binding binds exactly those.  No compute call is made (this runs without a GPU)."""

import os
import re

import ekv_hip

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "ekv_hip.h")


def declared() -> set[str]:
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:const\s+char\s*\*|int|size_t)\s*(ekv_\w+)\s*\(", text, re.M))


def test_header_declares_the_hot_path():
    names = declared()
    for name in ("ekv_audit_tile_lse", "ekv_tile_shares", "ekv_normalize_tile_lse", "ekv_rank_uniform",
                 "ekv_rank_uniform_ws", "ekv_compact_view", "ekv_build_view"):
        assert name in names


def test_binding_covers_the_header():
    assert set(ekv_hip.exported()) == declared()


def test_library_loads_and_exports_every_symbol():
    lib = ekv_hip.load()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.ekv_abi_version() == 1
    assert isinstance(lib.ekv_last_error(), bytes)


def test_argument_errors_map_to_value_error():
    # a null pointer is rejected by the argument checks before any device work
    try:
        ekv_hip.call("ekv_compact_view", 0, 0, 0, 0, 0, 1, 1, 16, 0, 0, 0, 0)
        raised = None
    except ValueError as err:
        raised = str(err)
    assert raised and "null" in raised
