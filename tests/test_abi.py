"""The C-ABI library loads on a GPU-less host and exports every entry point
declared in include/tf_hip.h; argument errors come back as tf_status codes
with a message, never as crashes.  No kernel is launched here."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions(header: Path) -> list[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tf_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions(ROOT / "include" / "tf_hip.h")
    assert "tf_gemm" in names and "tf_ce_bwd" in names and "tf_sgd_momentum" in names
    assert len(names) >= 40


def test_library_exports_every_declared_symbol():
    import tensors_amd._lib as L
    names = declared_functions(ROOT / "include" / "tf_hip.h")
    missing = [n for n in names if not hasattr(L.lib, n)]
    assert not missing, f"libtf_hip.so lacks: {missing}"
    # and the ctypes signature table covers them all
    assert set(names) - {"tf_last_error", "tf_version"} <= set(L.SIGNATURES)


def test_version_and_device_count():
    import tensors_amd as ta
    assert b"gfx950" in ta._lib.lib.tf_version()
    assert ta.device_count() >= 0


def test_null_context_is_rejected_with_message():
    import tensors_amd._lib as L
    st = L.lib.tf_relu_bwd(None, None, None, None, 4, L.TF_F32)
    assert st == L.TF_ERR_INVALID
    assert b"tf_ctx" in L.lib.tf_last_error()
    with pytest.raises(L.TFError):
        L.call("tf_hip_sync", None)


def test_init_without_gpu_fails_cleanly():
    import tensors_amd as ta
    import tensors_amd._lib as L
    if ta.device_count() > 0:
        pytest.skip("a GPU is visible; this checks the GPU-less path")
    h = C.c_void_p()
    st = L.lib.tf_hip_init(0, C.byref(h))
    assert st != L.TF_OK and h.value is None
    assert b"device" in L.lib.tf_last_error()
