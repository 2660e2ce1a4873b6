"""CPU checks of the C ABI: the library loads without a GPU and exports every
function include/dq8.h declares; argument errors are reported as statuses."""
import ctypes

import dq8


def test_library_loads_and_exports_every_declared_symbol():
    lib = dq8.lib()
    names = dq8.header_functions()
    assert len(names) >= 13
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_status_strings():
    assert dq8.status_string(dq8.OK) == "ok"
    assert dq8.status_string(dq8.ERR_NONFINITE) == "non-finite input"
    assert dq8.status_string(99) == "unknown status"


def test_null_arguments_are_rejected_without_touching_a_device():
    lib = dq8.lib()
    assert lib.dq8_create(0, None) == dq8.ERR_ARG
    assert lib.dq8_destroy(None) == dq8.ERR_ARG
    assert lib.dq8_weights_free(None) == dq8.ERR_ARG
    n, k = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.dq8_weights_shape(None, ctypes.byref(n), ctypes.byref(k)) == dq8.ERR_ARG
    assert lib.dq8_linear(None, None, None, None, 1, None, None, 0, 0, None) == dq8.ERR_ARG
    assert lib.dq8_linear_batch(None, None, 0, None) == dq8.ERR_ARG
    assert lib.dq8_quantize(None, None, 1, 1, None, None, None, None) == dq8.ERR_ARG
