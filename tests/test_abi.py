"""The C ABI library (no GPU needed): it loads, exports every entry point
include/ien_hip.h declares, and reports a missing device as IEN_ERR_GPU
(the reference's Error::Gpu, the signal to fall back to the CPU)."""

import ctypes
import re

import pytest

from conftest import ROOT


def declared():
    text = (ROOT / "include" / "ien_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ien_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    import ien

    lib = ctypes.CDLL(str(ien.LIB_PATH))
    names = declared()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(ien.EXPORTS)


def test_no_device_is_a_gpu_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import ien

    L = ien.load()
    h = ctypes.c_void_p()
    assert L.ien_open(0, ctypes.byref(h)) == ien.ERR_GPU
    assert L.ien_last_error().startswith(b"GPU: ")


def test_null_arguments_are_input_errors():
    import ien

    L = ien.load()
    assert L.ien_sync(None) == ien.ERR_INPUT
    assert L.ien_last_error().startswith(b"input: ")
    assert L.ien_model_set_graph(None, 1) == ien.ERR_INPUT


def test_descriptors_keep_their_tensor_alive():
    """An ien_input holds a raw pointer; the Python descriptor must keep the
    tensor behind it alive (a capture's empty_cache would otherwise return
    the freed block to the driver while a replay still reads it)."""
    import gc
    import weakref

    import torch

    import ien

    x = torch.zeros(64, 16, dtype=torch.float16)
    ref = weakref.ref(x)
    inp = ien.image_input(x, 4, 16, 16)
    rows = ien.rows_input(x, 16)
    del x
    gc.collect()
    assert ref() is not None and inp._tensor is ref() and rows._tensor is ref()
    del inp, rows
    gc.collect()
    assert ref() is None
