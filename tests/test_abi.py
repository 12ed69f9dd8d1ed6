"""The C-ABI library loads and exports every entry point include/mlxhip.h
declares; without a GPU, calls fail with BackendUnavailable (no fallback)."""
import ctypes as C
import os
import re
import subprocess

import pytest

from oxidizedmlx_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mlxhip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlxhip_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(abi.LIB_PATH):
        pytest.fail("libmlxhip.so is not built (run __graft_entry__.build())")
    return abi.load_library()


def test_header_and_prototype_table_agree():
    assert declared_functions() == sorted(abi.PROTOTYPES), \
        set(declared_functions()) ^ set(abi.PROTOTYPES)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", abi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\s[TW]\s(mlxhip_\w+)$", out, flags=re.M))
    missing = set(declared_functions()) - exported
    assert not missing, missing


def test_abi_version(lib):
    assert lib.mlxhip_abi_version() == abi.ABI_VERSION == 1


def test_struct_layouts():
    # x86-64 sizes of the C structs (checked against the C compiler below).
    assert C.sizeof(abi.mlxhip_op_t) == 112
    assert C.sizeof(abi.mlxhip_input_t) == 40
    assert C.sizeof(abi.mlxhip_meta_t) == 24
    assert C.sizeof(abi.mlxhip_ew_instr_t) == 8


def test_struct_layouts_match_compiler(tmp_path):
    src = tmp_path / "s.c"
    src.write_text('#include <stdio.h>\n#include "mlxhip.h"\nint main(void){printf("%zu %zu %zu %zu",'
                   'sizeof(mlxhip_op_t),sizeof(mlxhip_input_t),sizeof(mlxhip_meta_t),'
                   'sizeof(mlxhip_ew_instr_t));return 0;}\n')
    exe = tmp_path / "s"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    sizes = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()))
    assert sizes == [C.sizeof(abi.mlxhip_op_t), C.sizeof(abi.mlxhip_input_t),
                     C.sizeof(abi.mlxhip_meta_t), C.sizeof(abi.mlxhip_ew_instr_t)]


def test_free_null_is_noop(lib):
    lib.mlxhip_buffer_free(None)
    lib.mlxhip_stream_free(None)
    lib.mlxhip_event_destroy(None)


def test_null_arguments_rejected_without_gpu(lib):
    # Argument checks run before any device call.
    assert lib.mlxhip_eval_node(None, None, 0, None, None, 0) == abi.ERR_NULL_PTR
    assert lib.mlxhip_last_status() == abi.ERR_NULL_PTR
    assert b"null" in lib.mlxhip_last_error()


def test_no_gpu_means_backend_unavailable(lib):
    if lib.mlxhip_device_count() > 0:
        pytest.skip("a GPU is present")
    assert lib.mlxhip_init(0) == abi.ERR_BACKEND_UNAVAILABLE
    with pytest.raises(abi.BackendUnavailable):
        from oxidizedmlx_amd import backend
        backend.init()


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(abi.BackendUnavailable):
        abi.load_library(str(tmp_path / "nope.so"))


def test_shape_mismatch_payload_without_gpu(lib):
    # mlxhip_eval_node checks out_len against out_meta before any device call;
    # the failure carries MlxError::ShapeMismatch{expected, got}.
    from oxidizedmlx_amd.opkind import OpKind, meta
    cop, k1 = OpKind.Neg.to_c()
    cm, k2 = meta([2, 3]).to_c()
    out = (C.c_float * 5)()
    rc = lib.mlxhip_eval_node(C.byref(cop), None, 0, C.byref(cm), C.addressof(out), 5)
    assert rc == abi.ERR_SHAPE_MISMATCH
    assert abi.last_shape_mismatch(lib) == ([6], [5])
    with pytest.raises(abi.ShapeMismatch) as ei:
        abi.check(rc, lib)
    assert (ei.value.expected, ei.value.got) == ([6], [5])
    assert b"Shape mismatch: expected [6], got [5]" in lib.mlxhip_last_error()
    # Any other failure clears the payload.
    assert lib.mlxhip_eval_node(None, None, 0, None, None, 0) == abi.ERR_NULL_PTR
    assert abi.last_shape_mismatch(lib) is None
