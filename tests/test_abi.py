"""CPU-side checks of the boundary: the C-ABI library loads and exports every
entry point include/miburn.h declares (no compute call is made: there is no
GPU here), and the Python binding names every one of them."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "miburn.h")
LIB = os.path.join(ROOT, "metalium-rs_amd", "libmiburn.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_engine_surface():
    names = declared()
    for must in ("mi_ctx_create", "mi_upload", "mi_download", "mi_free", "mi_sync", "mi_matmul",
                 "mi_matmul_batched", "mi_eltwise", "mi_reduce", "mi_softmax_rows", "mi_rms_norm",
                 "mi_argmax_rows", "mi_select_rows", "mi_pick_columns", "mi_select_add_rows",
                 "mi_scatter_add_columns", "mi_cast", "mi_random", "mi_copy_strided"):
        assert must in names


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built")
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_header():
    import miburn
    src = open(miburn.__file__).read()
    missing = [n for n in declared() if n not in src]
    assert not missing, missing


def test_binding_fails_loudly_without_the_library(tmp_path, monkeypatch):
    import miburn
    monkeypatch.setattr(miburn, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(miburn, "_lib", None)
    with pytest.raises(ImportError):
        miburn.lib()


def test_context_create_without_gpu_reports_an_error():
    # No device in this container: creation must fail with a HIP status, not crash.
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import miburn
    with pytest.raises(miburn.MiError) as e:
        miburn.Engine(0)
    assert e.value.kind in ("HIP", "ARG")
