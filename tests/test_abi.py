"""CPU checks of the C-ABI library: it loads, exports every entry point that
include/fletcher_hip.h declares, and reports errors as status codes (no GPU
work is issued here)."""
import ctypes

import pytest


def test_header_declares_the_boundary(fl):
    syms = fl.header_symbols()
    # The Tensor / Backend methods on the hot path (device.go:5-162) and the
    # model-level ForwardBatch (bert.go:149-169).
    for s in ("fl_init", "fl_free_context", "fl_synchronize", "fl_vram_usage", "fl_alloc",
              "fl_free", "fl_gemm", "fl_linear", "fl_add_layernorm", "fl_layernorm",
              "fl_attention", "fl_attention_varlen", "fl_rope", "fl_gather_rows", "fl_cast",
              "fl_has_nan", "fl_mean_pool", "fl_model_create", "fl_model_forward",
              "fl_model_forward_device", "fl_model_set_weight"):
        assert s in syms


def test_library_exports_every_declared_symbol(fl):
    lib = fl.lib()
    missing = [s for s in fl.header_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert set(fl._SIGS) >= set(fl.header_symbols())


def test_error_path_without_context(fl):
    lib = fl.lib()
    assert lib.fl_synchronize(None) == fl.ERR_INVALID
    assert b"null context" in lib.fl_last_error()
    with pytest.raises(fl.FletcherError):
        fl.check(lib.fl_alloc(None, 16, ctypes.byref(ctypes.c_void_p())))
    assert lib.fl_version().startswith(b"fletcher-hip")
