"""The C ABI library loads and exports every entry point include/wavo_hip.h declares; error paths that
need no GPU (no device, bad arguments) report through wh_last_error.  No compute without a GPU."""

import ctypes
import os
import re

import pytest

import wavo_amd as wa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "wavo_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(wa.LIB_PATH)
    names = declared()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # The binding's signature table covers exactly the header.
    assert sorted(wa.SIGNATURES) == names


def test_binding_loads():
    assert wa.lib() is not None


def test_open_without_gpu_or_bad_index_is_a_gpu_error():
    # Here (no GPU) any index fails; on a GPU box an index past the devices fails the same way
    # (the reference's index_past_the_gpus, src/gpu/mod.rs:1712-1715).
    with pytest.raises(wa.WavoError) as e:
        wa.Gpu(1 << 20)
    assert e.value.fatal
    assert "GPU" in str(e.value) or "gfx950" in str(e.value)


def test_null_context_arguments_are_rejected():
    L = wa.lib()
    assert L.wh_sync(None) == wa.EARG
    assert L.wh_gemm(None, None, None, None, 1, 0, 0.0) == wa.EARG
    assert L.wh_linear_width(None) == 0
    assert L.wh_attend_len(4100, 2, 40) == 17 * 2 * 42
