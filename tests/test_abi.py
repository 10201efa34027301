"""The C ABI library loads and exports every entry point include/jevons_qmm.h declares, and its
host-only calls work without a GPU (no compute calls here)."""
import ctypes as C
import os

import pytest

import jevons_qmm as jq


def test_library_and_code_object_are_built():
    assert os.path.exists(jq.LIB_PATH), "run python jevons-rs_amd/build.py"
    assert os.path.exists(jq.HSACO_PATH)


def test_every_declared_symbol_is_exported():
    L = C.CDLL(jq.LIB_PATH)
    names = jq.header_symbols()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_type_table_matches_gguf():
    # gguf.rs:134-144
    assert jq.type_block(jq.Q4K) == (256, 144)
    assert jq.type_block(jq.Q6K) == (256, 210)
    assert jq.type_block(jq.Q8_0) == (32, 34)
    assert jq.type_block(jq.Q5_0) == (32, 22)
    assert jq.type_block(jq.F16) == (1, 2)
    assert jq.type_block(jq.F32) == (1, 4)
    assert jq.type_block(2) is None
    assert b"unsupported" in jq.lib().jv_last_error()


def test_code_object_targets_gfx950():
    data = open(jq.HSACO_PATH, "rb").read()
    assert data[:4] == b"\x7fELF"
    assert b"gfx950" in data
    for name in (b"jv_qmm_q4k_m1_n1", b"jv_qmm_q6k_m8_n4", b"jv_qmm_q8_0_m2_n1", b"jv_qmm_q5_0_m4_n2",
                 b"jv_qmm_f16_m8_n2", b"jv_argmax_partial", b"jv_argmax_final", b"jv_reduce_splits",
                 b"jv_repack_q6k", b"jv_dequant_q4k"):
        assert name in data, name


def test_open_fails_cleanly_without_a_gfx950_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    st = jq.lib().jv_open(0, C.byref(h))
    assert st != 0 and not h.value
    assert jq.lib().jv_last_error()
