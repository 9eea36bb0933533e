"""The C ABI library without a GPU: it loads, exports every function include/qmatmul.h declares (and the binding
describes each), and its host-only entry points answer. No kernel is launched here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    txt = open(os.path.join(ROOT, "include", "qmatmul.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(qmatmul_\w+)\s*\(", txt)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for n in ("qmatmul_gemv", "qmatmul_gemm", "qmatmul_moe_grouped", "qmatmul_quantize_act",
              "qmatmul_prepare_weight", "qmatmul_release_weight"):
        assert n in names


def test_library_exports_every_declared_symbol(qm):
    lib = qm.load_library()
    for n in declared_functions():
        assert hasattr(lib, n), n
    bound = {s[0] for s in qm.SIGNATURES}
    assert bound == set(declared_functions())


def test_host_only_entry_points(qm):
    lib = qm.load_library()
    assert lib.qmatmul_sb_bytes(8) == 272 and lib.qmatmul_sb_bytes(12) == 144
    assert lib.qmatmul_sb_bytes(21) == 110 and lib.qmatmul_sb_bytes(23) == 136 and lib.qmatmul_sb_bytes(6) == 0 and lib.qmatmul_sb_bytes(2) == 144
    assert lib.qmatmul_weight_bytes(23, 17408, 5120) >= 17408 * 20 * 136
    assert lib.qmatmul_weight_bytes(23, 16, 100) == 0
    # 32-element block types: rows of K % 32 == 0 are padded to whole superblocks (640 -> 768); others refuse them
    assert lib.qmatmul_weight_bytes(8, 16, 640) == lib.qmatmul_weight_bytes(8, 16, 768)
    assert lib.qmatmul_weight_bytes(20, 16, 640) == lib.qmatmul_weight_bytes(20, 16, 768) > 0
    assert lib.qmatmul_weight_bytes(23, 16, 640) == 0 and lib.qmatmul_weight_bytes(8, 16, 648) == 0
    assert lib.qmatmul_gemm_workspace_size(None, 128) == 0
    assert lib.qmatmul_moe_workspace_size(4096, 256, 8, 2048, 512) > 32768 * 2048 * 4
    L = qm.moe_ws_layout(4096, 256, 8, 2048, 512)
    assert L.slots == 32768 and L.max_tiles == 32768 // L.tile_rows + 2 * 256 and L.total >= L.y + 32768 * 2048 * 4


def test_argument_errors_need_no_gpu(qm):
    lib = qm.load_library()
    h = ctypes.c_void_p()
    # null source pointer / unsupported type / bad K: rejected before any device call
    assert lib.qmatmul_prepare_weight(23, None, 1, 16, 256, None, ctypes.byref(h)) == 1
    assert b"null" in lib.qmatmul_last_error()
    buf = (ctypes.c_uint8 * 16)()
    assert lib.qmatmul_prepare_weight(6, buf, 0, 16, 256, None, ctypes.byref(h)) == 3
    assert lib.qmatmul_prepare_weight(23, buf, 0, 16, 100, None, ctypes.byref(h)) == 2
    assert lib.qmatmul_prepare_weight(23, buf, 0, 16, 640, None, ctypes.byref(h)) == 2  # (IQ4_XS: whole superblocks)
    assert lib.qmatmul_gemm_ws(None, None, None, None, 1, 1, 1, None, 0, 0, 0, None, 0, None) == 1
    assert lib.qmatmul_gemv(None, None, None, None, 1, 1, None, 0, 0, 0, None) == 1
    assert lib.qmatmul_quantize_act(buf, 32, 1, 1, 33, buf, buf, buf, None) == 2
    # per-256 activation scales (act32 = 0) need K % 256 == 0; act32 is 0 or 1
    assert lib.qmatmul_quantize_act_ex(buf, 288, 1, 1, 288, 0, buf, buf, buf, None) == 2
    assert lib.qmatmul_quantize_act_ex(buf, 256, 1, 1, 256, 2, buf, buf, buf, None) == 1
    assert lib.qmatmul_swiglu_quant_ex(buf, 576, 288, 1, 1, 0, 0, 0, buf, buf, buf, None) == 2
    with pytest.raises(qm.QMatmulError):
        qm._call("qmatmul_moe_ws_layout", 0, 1, 1, 1, 1, None)


def test_type_table_agrees_across_header_binding_and_library(qm):
    """Every qm_type of the header has the GGML id the Python formats use, and the library reports the GGUF bytes per
    256 elements the formats module (and ggml's block structs) give it."""
    from arcinfer_amd import formats as F
    txt = open(os.path.join(ROOT, "include", "qmatmul.h")).read()
    ids = {k: int(v) for k, v in re.findall(r"\bQM_((?:I?Q)\w+?)\s*=\s*(\d+)", txt)}
    assert len(ids) == 17
    lib = qm.load_library()
    for name, tid in ids.items():
        assert getattr(F, name) == tid, name
        assert lib.qmatmul_sb_bytes(tid) == F.SB_BYTES[tid], name
    # rows: whole superblocks, except the 32-element block types (any K % 32 == 0, padded) and Q2_0 (K % 64 == 0)
    for tid in ids.values():
        ok640 = lib.qmatmul_weight_bytes(tid, 16, 640) > 0
        assert ok640 == (tid in (F.Q8_0, F.Q4_0, F.IQ4_NL, F.Q2_0)), tid
    assert lib.qmatmul_weight_bytes(F.Q2_0, 16, 608) == 0 and lib.qmatmul_weight_bytes(F.Q8_0, 16, 608) > 0
