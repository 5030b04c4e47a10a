"""The Python locator keeps the reference surface (src/colabfold_legacy_kernels/__init__.py:1-92)
and the reference CI smoke test (.github/workflows/build-and-publish.yml:72-90), with gfx950 in
place of sm_70/sm_75."""
import ctypes
from pathlib import Path

import pytest

import colabfold_legacy_kernels as clk


def test_public_names():
    assert set(clk.__all__) == {"KERNELS", "available", "kernel_dir", "library_path",
                                "supported_capabilities", "symbol"}
    assert clk.KERNELS[:3] == ("attention", "layer_norm", "gated_dual_proj")
    assert clk.supported_capabilities() == ("gfx950",)


def test_reference_targets_keep_their_names():
    assert clk.symbol("attention", "gfx950") == "VoltaMma"
    assert clk.symbol("layer_norm", 950) == "VoltaLayerNorm"
    assert clk.symbol("gated_dual_proj", "950") == "VoltaGdp"


def test_unknown_kernel_raises_key_error():
    with pytest.raises(KeyError):
        clk.symbol("softmax", "gfx950")
    with pytest.raises(KeyError):
        clk.library_path("softmax", "gfx950")
    assert clk.available("gfx950", "softmax") is False


@pytest.mark.parametrize("cc", [70, 75, 80, 90, "gfx942", "gfx1100"])
def test_other_architectures_have_no_library(cc):
    assert clk.available(cc) is False
    with pytest.raises(FileNotFoundError):
        clk.library_path("attention", cc)
    with pytest.raises(FileNotFoundError):
        clk.symbol("attention", cc)


def test_kernel_dir():
    assert Path(clk.kernel_dir("gfx950")).name == "gfx950"
    assert Path(clk.kernel_dir(75)).name == "sm75"


def test_missing_library_is_reported(monkeypatch, tmp_path):
    monkeypatch.setattr(clk, "_KERNEL_DIR", tmp_path)
    assert clk.available("gfx950") is False
    with pytest.raises(FileNotFoundError):
        clk.library_path("attention", "gfx950")
    assert clk.symbol("attention", "gfx950") == "VoltaMma"


@pytest.mark.skipif(not clk.available("gfx950"), reason="library not built")
def test_ci_smoke():
    """build-and-publish.yml:79-88 with gfx950: every kernel's library loads and its FFI symbol
    resolves; a CUDA capability (sm_80) reports unavailable."""
    assert clk.available("gfx950")
    for kernel in clk.KERNELS:
        assert clk.available("gfx950", kernel)
        lib = ctypes.cdll.LoadLibrary(clk.library_path(kernel, "gfx950"))
        getattr(lib, clk.symbol(kernel, "gfx950"))
    assert not clk.available(80)
