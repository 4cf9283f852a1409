"""CPU checks of the C ABI: libmmnb.so loads, exports every function
include/mmnb.h declares, and rejects bad arguments before touching a device.
No compute call is made here (no GPU in this environment)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from onnx_runtime_dart_amd import _lib, ops

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mmnb.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mmnb_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_operator_entry_points():
    names = declared_functions()
    for fn in ["mmnb_pack_nbits", "mmnb_matmul_nbits", "mmnb_matmul_nbits_dev",
               "mmnb_dynamic_quantize_linear", "mmnb_dynamic_quantize_linear_dev",
               "mmnb_pack_integer", "mmnb_matmul_integer", "mmnb_matmul_integer_dev",
               "mmnb_dynamic_matmul_dev", "mmnb_pack_free", "mmnb_last_error"]:
        assert fn in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_abi_version():
    assert _lib.load().mmnb_abi_version() == 1


def test_null_context_is_argument_error():
    lib = _lib.load()
    h = ctypes.c_void_p()
    rc = lib.mmnb_pack_nbits(None, None, 0, None, 0, None, 0, 32, 1, 4, 32,
                             ctypes.byref(h))
    assert rc == _lib.MMNB_ERR_ARG
    assert b"null context" in lib.mmnb_last_error()
    with pytest.raises(ValueError):
        _lib.check(rc)


def test_init_without_a_gpu_reports_device_error_or_succeeds():
    # Here (no GPU) mmnb_init must fail cleanly with a device error and a
    # message, never crash.  On a GPU host it succeeds.
    lib = _lib.load()
    h = ctypes.c_void_p()
    rc = lib.mmnb_init(0, ctypes.byref(h))
    if rc == 0:
        assert lib.mmnb_shutdown(h) == 0
    else:
        assert rc == _lib.MMNB_ERR_DEVICE
        assert lib.mmnb_last_error()


def test_status_codes_map_to_reference_exception_types():
    lib = _lib.load()
    lib.mmnb_pack_nbits(None, None, 0, None, 0, None, 0, 32, 1, 4, 32,
                        ctypes.byref(ctypes.c_void_p()))
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.MMNB_ERR_UNSUPPORTED)
    with pytest.raises(MemoryError):
        _lib.check(_lib.MMNB_ERR_OOM)
    with pytest.raises(_lib.MmnbError):
        _lib.check(_lib.MMNB_ERR_DEVICE)


def test_dispatch_rejects_extra_matmulnbits_inputs_before_any_device_call():
    # onnx_graph.dart:1585-1588: g_idx / bias inputs -> UnsupportedError
    with pytest.raises(NotImplementedError, match="g_idx"):
        ops.dispatch("MatMulNBits", [np.zeros((1, 32), np.float32)] * 5,
                     {"K": 32, "N": 1, "bits": 4, "block_size": 32})


def test_dispatch_rejects_bits_other_than_4_before_any_device_call():
    # onnx_qlinear_ops.dart:117-119
    with pytest.raises(NotImplementedError, match="bits=4"):
        ops.op_matmul_nbits(np.zeros((1, 32), np.float32), np.zeros((1, 1, 16), np.uint8),
                            np.ones(1, np.float32), None, k=32, n=1, bits=8,
                            block_size=32)


def test_unknown_op_is_unsupported():
    with pytest.raises(NotImplementedError):
        ops.dispatch("QLinearAdd", [], {})


def test_missing_required_input_is_an_argument_error():
    with pytest.raises(ValueError):
        ops.dispatch("QLinearConv", [], {})
