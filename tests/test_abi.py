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


COMPUTE = ("ekv_audit_tile_lse", "ekv_tile_shares", "ekv_tile_shares_ws", "ekv_tile_shares_noalloc", "ekv_normalize_tile_lse",
           "ekv_rank_uniform", "ekv_rank_uniform_ws", "ekv_rank_uniform_view", "ekv_rank_sum", "ekv_rank_maxmin", "ekv_compact_view",
           "ekv_build_view", "ekv_compact_slots", "ekv_controller_keep", "ekv_audit_stage_queries")


def test_every_entry_point_rejects_null_pointers_on_the_host():
    # null pointers with zero sizes: each entry point's argument checks refuse them (ValueError)
    # before any device call, which is why this runs without a GPU
    import pytest

    lib = ekv_hip.load()
    for name in COMPUTE:
        args = [0] * len(getattr(lib, name).argtypes)
        with pytest.raises(ValueError):
            ekv_hip.call(name, *args)


def test_shape_limits_are_refused_on_the_host():
    import pytest

    P = 256  # a placeholder device address: the checks below refuse the call before using it
    # ranking: a row wider than the streaming kernel's LDS holds (262144 blocks)
    wide = 300000
    with pytest.raises(ValueError, match="width"):
        ekv_hip.call("ekv_rank_uniform", P, wide, P, 0, 0, 0, 0, 0, 0, 0, 4, wide, 0.5, -1, P, wide, 0, 0)
    # ranking + view: the same width limit, and a block size below 1
    with pytest.raises(ValueError, match="width"):
        ekv_hip.call("ekv_rank_uniform_view", P, wide, P, 0, 0, 0, 4, wide, 0.5, -1, P, wide, 0, P, wide, P, 16,
                     P, wide, P, 0, 0)
    with pytest.raises(ValueError, match="block size"):
        ekv_hip.call("ekv_rank_uniform_view", P, 64, P, 0, 0, 0, 4, 64, 0.5, -1, P, 64, 0, P, 64, P, 0, P, 64, P, 0, 0)
    # sum and maxmin: rows past 262144 blocks
    with pytest.raises(ValueError, match="width"):
        ekv_hip.call("ekv_rank_sum", P, wide, P, 0, 0, 0, 4, wide, 10, P, wide, 0, P, 1 << 20, 0)
    with pytest.raises(ValueError, match="width"):
        ekv_hip.call("ekv_rank_maxmin", P, wide, P, 0, 0, 4, wide, 10, P, wide, 0, P, 1 << 20, 0)
    # maxmin: a workspace below the size the call reports (no 32-bit limit on rows x width)
    need = int(ekv_hip.load().ekv_rank_maxmin_workspace(8192, 262144))
    with pytest.raises(ValueError, match="workspace"):
        ekv_hip.call("ekv_rank_maxmin", P, 262144, P, 0, 0, 8192, 262144, 10, P, 262144, 0, P, need - 4096, 0)
    # sum and maxmin: 2^24 requests or more
    with pytest.raises(ValueError, match="rows"):
        ekv_hip.call("ekv_rank_maxmin", P, 8, P, 0, 0, 1 << 24, 8, 10, P, 8, 0, P, 1 << 30, 0)
    with pytest.raises(ValueError, match="rows"):
        ekv_hip.call("ekv_rank_sum", P, 8, P, 0, 0, 0, 1 << 24, 8, 10, P, 8, 0, P, 1 << 30, 0)
    with pytest.raises(ValueError, match="width"):
        ekv_hip.call("ekv_controller_keep", ekv_hip.OBJ_MAXMIN, P, ekv_hip.F64, wide, P, P, 0, 0, 0, 0, 4, wide,
                     4, 0, 0.5, P, wide, 0, P, 1 << 30, 0)
    # ranking: explicit masks without a workspace
    with pytest.raises(ValueError, match="workspace"):
        ekv_hip.call("ekv_rank_uniform", P, 8, P, 0, P, 8, 0, 0, 0, 0, 4, 8, 0.5, -1, P, 8, 0, 0)
    # audit: more query rows per KV head than a record holds
    audit = [P, ekv_hip.BF16, 4096, 128, P, ekv_hip.BF16, 65536, 1024, 128, 1.0, P, 8, P, P, P, P,
             P, 1 << 20, 1 << 16, 64, 17, 0, 0, 0.1, 0, 0, 1, 17, 4, 8, 16, 2, 128, 0, 0]
    with pytest.raises(ValueError, match="query rows"):
        ekv_hip.call("ekv_audit_tile_lse", *audit)
    # audit: tiles of another number of blocks than the records hold
    audit[20], audit[27], audit[31] = 4, 4, 3
    with pytest.raises(ValueError, match="tiles"):
        ekv_hip.call("ekv_audit_tile_lse", *audit)
    # SGLang lists: slots of 3 bytes
    with pytest.raises(ValueError, match="slots"):
        ekv_hip.call("ekv_compact_slots", P, P, 3, P, 8, 0, 1, 1, 1, 8, 16, 16, P, P, P, 8, P, 0, 0, 0)
    # the controller's rule: an unknown objective, weights under maxmin, a fraction outside (0, 1]
    ctl = [ekv_hip.OBJ_SUM, P, ekv_hip.F32, 64, P, P, 0, 0, 0, 0, 4, 64, 1, 0, 0.5, P, 64, 0, P, 1 << 30, 0]
    for at, value, match in ((0, 7, "objective"), (9, P, "weights"), (14, 1.5, "fraction"), (14, 0.0, "fraction")):
        bad = list(ctl)
        bad[at] = value
        if at == 9:
            bad[0] = ekv_hip.OBJ_MAXMIN
        with pytest.raises(ValueError, match=match):
            ekv_hip.call("ekv_controller_keep", *bad)


def test_the_multi_layer_audit_refuses_bad_layer_lists_on_the_host():
    import pytest

    lib = ekv_hip.load()
    args = [0] * len(lib.ekv_audit_tile_lse_layers.argtypes)
    args[0] = None
    args[1] = 1
    with pytest.raises(ValueError, match="layer list"):
        ekv_hip.call("ekv_audit_tile_lse_layers", *args)
    # a query type the keys do not pair with, and a null table, refused before any launch
    one = (ekv_hip.AuditLayer * 1)(ekv_hip.AuditLayer(256, 256, 0, 0, 0, 1.0, 1.0, 0))
    P = 256
    args = [one, 1, 1, ekv_hip.F16, 512, 128, ekv_hip.BF16, 1 << 16, 1024, 128, P, 8, P, P, P, P, P, 1 << 20, 1 << 16,
            64, 4, 0, 0, 1, 4, 4, 8, 16, 2, 128, P, 1 << 20, 4, 8, 0]
    with pytest.raises(ValueError, match="not supported"):
        ekv_hip.call("ekv_audit_tile_lse_layers", *args)
    args[3] = ekv_hip.BF16
    args[10] = 0
    with pytest.raises(ValueError, match="null"):
        ekv_hip.call("ekv_audit_tile_lse_layers", *args)


def test_audit_shapes():
    lib = ekv_hip.load()
    both = ekv_hip.AUDIT_SELF_CONTAINED | ekv_hip.AUDIT_PLANNED
    assert lib.ekv_audit_shape(ekv_hip.BF16, ekv_hip.BF16, 128, 16) == both
    assert lib.ekv_audit_shape(ekv_hip.BF16, ekv_hip.FP8_E4M3, 128, 32) == both
    assert lib.ekv_audit_shape(ekv_hip.F16, ekv_hip.F16, 64, 16) == both
    assert lib.ekv_audit_shape(ekv_hip.BF16, ekv_hip.BF16, 32, 16) == both  # MFMA at 32 dimensions
    assert lib.ekv_audit_shape(ekv_hip.F32, ekv_hip.F32, 128, 16) == both  # the VALU forms
    assert lib.ekv_audit_shape(ekv_hip.BF16, ekv_hip.BF16, 128, 8) == both
    # the VALU shapes only a step plan takes: 32 or 256 dimensions on the VALU, small rows in 8-token blocks
    for q, k, d, bs in ((ekv_hip.F32, ekv_hip.F32, 32, 16), (ekv_hip.F32, ekv_hip.F32, 256, 8),
                        (ekv_hip.BF16, ekv_hip.BF16, 256, 8), (ekv_hip.BF16, ekv_hip.FP8_E4M3, 64, 8),
                        (ekv_hip.BF16, ekv_hip.FP8_E4M3, 32, 16), (ekv_hip.BF16, ekv_hip.FP8_E4M3, 32, 8),
                        (ekv_hip.BF16, ekv_hip.BF16, 32, 8)):
        assert lib.ekv_audit_shape(q, k, d, bs) & ekv_hip.AUDIT_PLANNED, (q, k, d, bs)
    assert lib.ekv_audit_shape(ekv_hip.F16, ekv_hip.BF16, 128, 16) == 0  # mixed 16-bit types
    assert lib.ekv_audit_shape(ekv_hip.BF16, ekv_hip.BF16, 96, 16) == 0  # rows of 192 bytes
    assert lib.ekv_audit_shape(ekv_hip.BF16, ekv_hip.BF16, 128, 12) == 0  # tiles of 24 tokens
