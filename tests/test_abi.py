"""The C-ABI library loads and exports every entry point include/hobby_gpu.h declares, and the
Python mirror binds exactly that list.  No GPU needed: nothing here calls into HIP."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "hobby_gpu.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hg_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_boundary():
    names = _declared()
    for must in ("hg_model_load", "hg_forward", "hg_forward_x", "hg_prefill", "hg_kv_new",
                 "hg_q8_tensor_matvec", "hg_attention_decode", "hg_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import hobbylm_amd
    if not os.path.exists(hobbylm_amd.LIB_PATH):
        pytest.fail("libhobby_gpu.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(hobbylm_amd.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name
    assert sorted(hobbylm_amd.SIGNATURES) == _declared()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import hobbylm_amd
    monkeypatch.setattr(hobbylm_amd, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(hobbylm_amd, "_lib", None)
    with pytest.raises(ImportError, match="no CPU fallback"):
        hobbylm_amd.lib()
