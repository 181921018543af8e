"""The C-ABI library loads and exports every entry point the header declares;
argument validation runs on the host (no GPU calls)."""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest
import torch

from myelin_amd import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "myelin_hip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(myelin_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_entry_points():
    names = declared_functions()
    assert "myelin_last_error" in names and "myelin_abi_version" in names
    assert set(_lib.SIGNATURES) <= set(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.myelin_abi_version() == 1


def test_validation_errors_are_reported_without_launching():
    lib = _lib.load()
    rc = lib.myelin_lif_fwd_f32(None, None, None, None, None, None, 0, 1, 1, 0.9, 1.0, 0.0, 10.0, 0, 16, None)
    assert rc == _lib.EINVAL
    assert b"positive" in lib.myelin_last_error()
    with pytest.raises(ValueError, match="chunk must be 8 or 16"):
        _lib.call("myelin_lif_bwd_f32", 1, 1, None, None, 1, 1, 4, 4, 0.9, 1.0, 0.0, 10.0, 1, 12, None)
    with pytest.raises(ValueError, match="unknown surrogate"):
        _lib.call("myelin_alif_bwd_f32", 1, 1, 1, None, None, None, 1, 1, 1, 4, 4, 0.9, 0.9, 1.0, 1.8, 0.0,
                  10.0, 42, 16, None)
    with pytest.raises(ValueError, match="unsupported dtype"):
        _lib.call("myelin_pack", 1, 99, 1, 4, 4, None)
    with pytest.raises(ValueError, match="exactly one of spikes"):
        _lib.call("myelin_lif_fwd_f32", 1, 1, 1, 1, 1, None, 4, 1, 1, 0.9, 1.0, 0.0, 10.0, 0, 16, None)
    # empty problems are valid no-ops
    assert lib.myelin_pack(None, 0, None, 0, 5, None) == 0


def test_autograd_order_codes_are_validated_without_launching():
    st = _lib.RULE_STRAIGHT_THROUGH + 1
    # spike values cannot be packed into bits
    with pytest.raises(ValueError, match="packed output takes the threshold rules"):
        _lib.call("myelin_lif_fwd_f32", 1, 1, 1, None, 1, None, 4, 1, 1, 0.9, 1.0, 0.0, 10.0, st, 16, None)
    # the autograd rules exist for surrogate ids 0-5 only
    with pytest.raises(ValueError, match="unknown spike rule 22"):
        _lib.call("myelin_lif_fwd_f32", 1, 1, 1, 1, None, None, 4, 1, 1, 0.9, 1.0, 0.0, 10.0,
                  _lib.RULE_STRAIGHT_THROUGH + _lib.SG_NONE, 16, None)
    with pytest.raises(ValueError, match="unknown surrogate code 22"):
        _lib.call("myelin_lif_bwd_f32", 1, 1, None, None, 1, 1, 4, 4, 0.9, 1.0, 0.0, 10.0,
                  _lib.SG_AUTOGRAD + _lib.SG_NONE, 16, None)
    # the autograd-order backwards are built at chunk 16 only
    for code in (_lib.SG_AUTOGRAD_SMOOTH + 1, _lib.SG_AUTOGRAD + 1):
        with pytest.raises(ValueError, match="needs chunk 16"):
            _lib.call("myelin_alif_bwd_f32", 1, 1, 1, None, None, None, 1, 1, 1, 4, 4, 0.9, 0.9, 1.0, 1.8, 0.0,
                      10.0, code, 8, None)
        with pytest.raises(ValueError, match="needs chunk 16"):
            _lib.call("myelin_lif_bwd_f32", 1, 1, None, None, 1, 1, 4, 4, 0.9, 1.0, 0.0, 10.0, code, 8, None)


def test_error_message_is_per_thread():
    import threading

    lib = _lib.load()
    lib.myelin_pack(None, 0, None, -1, 5, None)
    seen = {}

    def worker():
        seen["msg"] = lib.myelin_last_error()

    th = threading.Thread(target=worker)
    th.start()
    th.join()
    assert seen["msg"] == b""
    assert b"rows" in lib.myelin_last_error()


def test_ctypes_signatures_match_header_arity():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, argtypes in _lib.SIGNATURES.items():
        m = re.search(rf"int {name}\((.*?)\);", text, flags=re.S)
        assert m, name
        assert len(m.group(1).split(",")) == len(argtypes), name


def test_pointer_types_are_plain():
    # the ABI takes void* / c types only: ctypes argtypes never name torch
    for argtypes in _lib.SIGNATURES.values():
        for a in argtypes:
            assert a in (ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int, ctypes.c_uint32)
    assert torch is not None


def test_gemm_workspace_size_is_host_only_and_covers_the_split():
    lib = _lib.load()
    # 784 x 2048 output over K = 12800: 112 tiles of 128 x 128 would split 5
    # ways; the 32 tiles of 256 x 256 that mn-contiguous bf16 operands take
    # split 8 ways, and the workspace covers the larger
    assert lib.myelin_gemm_workspace_elems(784, 2048, 12800, _lib.PREC["bf16"]) == 8 * 784 * 2048
    assert lib.myelin_gemm_workspace_elems(784, 2048, 12800, _lib.PREC["fp32"]) == 5 * 784 * 2048
    # enough tiles, or a short K: no split, no workspace
    assert lib.myelin_gemm_workspace_elems(12800, 2048, 784, _lib.PREC["bf16"]) == 0
    assert lib.myelin_gemm_workspace_elems(784, 2048, 100, _lib.PREC["fp32"]) == 0
    assert lib.myelin_gemm_workspace_elems(0, 5, 5, 0) == 0


def test_split_synapse_entry_points_validate_on_the_host():
    with pytest.raises(ValueError, match="parts must be in"):
        _lib.call("myelin_gemm_parts", 16, 16, 0, 0, None, 16, 4, 4, 4, 4, 4, 4, 0, 0, 0, None, 0, None)
    with pytest.raises(ValueError, match="parts must be in"):
        _lib.call("myelin_gemm_parts", 16, 16, 9, 64, None, 16, 4, 4, 4, 4, 4, 4, 0, 0, 0, None, 0, None)
    with pytest.raises(ValueError, match="16-byte"):  # k-contiguous A rows of 4 bf16 are 8 bytes
        _lib.call("myelin_gemm_parts", 16, 16, 3, 64, None, 16, 4, 4, 4, 4, 4, 4, 0, 0, 0, None, 0, None)
    with pytest.raises(ValueError, match="bad leading dim"):
        _lib.call("myelin_gemm_parts", 16, 16, 3, 64, None, 16, 4, 4, 8, 4, 4, 4, 0, 0, 0, None, 0, None)
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("myelin_cast_bf16_checked", 16, 16, 8, None, None)
    with pytest.raises(ValueError, match="16-byte aligned"):
        _lib.call("myelin_cast_bf16_checked", 4, 16, 8, 16, None)
    with pytest.raises(ValueError, match="negative size"):
        _lib.call("myelin_split_bf16x3", 16, 16, -1, 4, 0, None)
    with pytest.raises(ValueError, match="G must be float32, bfloat16 or three"):
        _lib.call("myelin_linear_pre_bwd", 16, None, None, 16, 16, 99, None, 4, 4, 4, 0.9, 1.0, 0.0, 5.0, 1, 0,
                  None)
    # the spike-gradient-forming reverse pass: O, N, C x O and G's type
    ro = ("myelin_linear_pre_bwd_readout", 16, 16, 16)
    tail = (0.9, 1.0, 0.0, 5.0, 1, 0, None)
    with pytest.raises(ValueError, match="O must be in"):
        _lib.call(*ro, 33, 16, 16, 0, None, 4, 2, 256, *tail)
    with pytest.raises(ValueError, match="multiple of 256"):
        _lib.call(*ro, 20, 16, 16, 0, None, 4, 2, 200, *tail)
    with pytest.raises(ValueError, match="G must be float32 or three"):
        _lib.call(*ro, 20, 16, 16, _lib.DT[torch.bfloat16], None, 4, 2, 256, *tail)
    with pytest.raises(ValueError, match="too large for the staged rows"):
        _lib.call(*ro, 20, 16, 16, 0, None, 820, 2, 256, *tail)
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("myelin_linear_pre_bwd_readout", 16, 16, None, 20, 16, 16, 0, None, 4, 2, 256, *tail)
    with pytest.raises(ValueError, match="unknown surrogate"):
        _lib.call(*ro, 20, 16, 16, 0, None, 4, 2, 256, 0.9, 1.0, 0.0, 5.0, 99, 0, None)
    # the GEMMs with an attached column sum, and the merged bf16 copies
    g = ("myelin_gemm_col_sum", 16, 0, 16, 0, None, 16, 4, 4, 4, 4, 4, 4, 0, 0, 0, 0, None, 0)
    with pytest.raises(ValueError, match="col_sum: negative size"):
        _lib.call(*g, 16, 16, -1, 4, None)
    with pytest.raises(ValueError, match="col_sum: null pointer"):
        _lib.call(*g, 16, None, 3, 4, None)
    with pytest.raises(ValueError, match="gemm: ldc < N"):
        _lib.call("myelin_gemm_col_sum", 16, 0, 16, 0, None, 16, 4, 4, 4, 4, 4, 3, 0, 0, 0, 0, None, 0, 16, 16, 3, 4,
                  None)
    with pytest.raises(ValueError, match="col_sum: null pointer"):
        _lib.call("myelin_gemm_parts_col_sum", 16, 16, 3, 64, None, 16, 4, 4, 8, 8, 4, 4, 0, 0, 0, None, 0, None, 16,
                  2, 4, None)
    with pytest.raises(ValueError, match="cast_transpose_bf16: negative size"):
        _lib.call("myelin_cast_transpose_bf16", 16, 16, -8, 16, 16, 4, 4, None)
    with pytest.raises(ValueError, match="16-byte aligned"):
        _lib.call("myelin_cast_transpose_bf16", 4, 16, 8, 16, 16, 4, 4, None)
    # empty problems are valid no-ops
    assert _lib.load().myelin_cast_transpose_bf16(None, None, 0, None, None, 0, 5, None) == 0
    assert _lib.load().myelin_gemm_col_sum(None, 0, None, 0, None, None, 0, 4, 4, 4, 4, 4, 0, 0, 0, 0, None, 0,
                                           None, None, 0, 0, None) == 0
    assert _lib.load().myelin_split_bf16x3(None, None, 0, 5, 1, None) == 0
    assert _lib.load().myelin_gemm_parts(None, None, 3, 0, None, None, 0, 4, 4, 4, 4, 4, 0, 0, 0, None, 0,
                                         None) == 0


def test_narrow_one_launch_entry_validates_on_the_host():
    nb = "myelin_linear_lif_fwd_narrow_bits"
    # words, w, bias, m0, m_final, spikes, pre, rates, T, B, F, N, t0, t1, decay, thr, reset, slope, rule, prec
    with pytest.raises(ValueError, match="at most 32 neurons"):
        _lib.call(nb, 16, 16, None, None, None, None, 16, None, 4, 4, 8, 33, 0, 4, 0.9, 1.0, 0.0, 10.0, 0, 1, None)
    with pytest.raises(ValueError, match="words and w are required"):
        _lib.call(nb, None, 16, None, None, None, None, 16, None, 4, 4, 8, 4, 0, 4, 0.9, 1.0, 0.0, 10.0, 0, 1, None)
    with pytest.raises(ValueError, match="whole range"):
        _lib.call(nb, 16, 16, None, None, None, None, None, 16, 4, 4, 8, 4, 1, 4, 0.9, 1.0, 0.0, 10.0, 0, 1, None)
    with pytest.raises(ValueError, match="bad time range"):
        _lib.call(nb, 16, 16, None, None, None, None, 16, None, 4, 4, 8, 4, 3, 3, 0.9, 1.0, 0.0, 10.0, 0, 1, None)
    with pytest.raises(ValueError, match="unknown rule"):
        _lib.call(nb, 16, 16, None, None, None, None, 16, None, 4, 4, 8, 4, 0, 4, 0.9, 1.0, 0.0, 10.0, 17, 1, None)
    with pytest.raises(ValueError, match="precision must be"):
        _lib.call(nb, 16, 16, None, None, None, None, 16, None, 4, 4, 8, 4, 0, 4, 0.9, 1.0, 0.0, 10.0, 0, 2, None)


def test_narrow_one_launch_size_query_is_host_only():
    lib = _lib.load()
    # the 2048 -> 10 bf16 readout fits (91,552 bytes of LDS), its fp32
    # form (three W planes) does not; 2048 -> 5 at fp32 does; the 4096 -> 20
    # fp32 readout does not; no layer over 32 neurons or with a bad precision
    assert lib.myelin_narrow_bits_fits(2048, 10, _lib.PREC["bf16"]) == 1
    assert lib.myelin_narrow_bits_fits(2048, 10, _lib.PREC["fp32"]) == 0
    assert lib.myelin_narrow_bits_fits(2048, 5, _lib.PREC["fp32"]) == 1
    assert lib.myelin_narrow_bits_fits(4096, 20, _lib.PREC["fp32"]) == 0
    assert lib.myelin_narrow_bits_fits(100, 33, _lib.PREC["bf16"]) == 0
    assert lib.myelin_narrow_bits_fits(100, 10, 2) == 0
    assert lib.myelin_narrow_bits_fits(0, 10, 1) == 0
