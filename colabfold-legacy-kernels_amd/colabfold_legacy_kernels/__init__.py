"""ColabFold Evoformer kernels for AMD Instinct MI355X (gfx950).

Drop-in counterpart of the ``colabfold_legacy_kernels`` locator
(src/colabfold_legacy_kernels/__init__.py:1-92): the same names, arguments, exceptions and
return values. It maps (kernel, architecture) to the shared library that holds the kernel and
to the XLA FFI target name that library exports; it loads nothing itself.

Differences, all supersets of the reference contract:
  * the architecture is ``"gfx950"`` (``950`` and ``"950"`` are accepted too); the CUDA
    capabilities 70/75/80 resolve to no library, so ``available(75)`` is False on this build;
  * the three reference kernels keep their FFI target names (VoltaMma, VoltaLayerNorm,
    VoltaGdp), so a caller that registers ``symbol(kernel, cc)`` needs no change;
  * three kernels the reference lacks are added: the attention backward, the LayerNorm backward
    and LayerNorm fused with both gated-projection branches.
"""

from pathlib import Path

__all__ = [
    "KERNELS",
    "available",
    "kernel_dir",
    "library_path",
    "supported_capabilities",
    "symbol",
]

__version__ = "0.2.0+gfx950"

_KERNEL_DIR = Path(__file__).resolve().parent / "kernels"

_ARCH = "gfx950"
_CAPABILITIES = (_ARCH,)
_LIB = "libclk_gfx950.so"

# kernel -> ((architecture, library, FFI target), ...), like _TABLE at __init__.py:21-33.
_TABLE = {
    "attention": ((_ARCH, _LIB, "VoltaMma"),),
    "layer_norm": ((_ARCH, _LIB, "VoltaLayerNorm"),),
    "gated_dual_proj": ((_ARCH, _LIB, "VoltaGdp"),),
    "attention_fwd_lse": ((_ARCH, _LIB, "ClkAttentionFwd"),),
    "attention_bwd": ((_ARCH, _LIB, "ClkAttentionBwd"),),
    "layer_norm_bwd": ((_ARCH, _LIB, "ClkLayerNormBwd"),),
    "ln_gated_dual_proj": ((_ARCH, _LIB, "ClkLnGdp"),),
    "attention_gate": ((_ARCH, _LIB, "ClkAttentionGate"),),
    "ln_pair_bias": ((_ARCH, _LIB, "ClkLnPairBias"),),
    "gated_dual_proj_bwd": ((_ARCH, _LIB, "ClkGdpBwd"),),
    "triangle_multiply": ((_ARCH, _LIB, "ClkTriangleMultiply"),),
}

KERNELS = tuple(_TABLE)


def supported_capabilities():
    """Give the architectures that this package contains."""
    return _CAPABILITIES


def _normalise(cc):
    """``"gfx950"``, ``950`` and ``"950"`` name gfx950; any other number stays a number."""
    if isinstance(cc, str) and cc.strip().lower().startswith("gfx"):
        return cc.strip().lower()
    cc = int(cc)
    return _ARCH if cc == 950 else cc


def _resolve(kernel, cc):
    """Find the library and the FFI symbol for one kernel and one architecture."""
    if kernel not in _TABLE:
        raise KeyError(
            "unknown kernel %r, expected one of %s" % (kernel, ", ".join(KERNELS)))
    cc = _normalise(cc)
    if cc not in _CAPABILITIES:
        return cc, None, None
    for arch, lib, sym in _TABLE[kernel]:
        if cc == arch:
            return cc, lib, sym
    return cc, None, None


def _dirname(cc):
    return cc if isinstance(cc, str) else "sm%d" % cc


def kernel_dir(cc):
    """Give the directory of the libraries for one architecture."""
    cc, _, _ = _resolve("attention", cc)
    return str(_KERNEL_DIR / _dirname(cc))


def library_path(kernel, cc):
    """Give the path of the library that supplies one kernel."""
    cc, lib, _ = _resolve(kernel, cc)
    if lib is None:
        raise FileNotFoundError("no %s kernel for architecture %s" % (kernel, cc))
    path = _KERNEL_DIR / _dirname(cc) / lib
    if not path.is_file():
        raise FileNotFoundError("%s is not in this package" % path)
    return str(path)


def symbol(kernel, cc):
    """Give the XLA FFI target name that the library exports."""
    cc, lib, sym = _resolve(kernel, cc)
    if sym is None:
        raise FileNotFoundError("no %s kernel for architecture %s" % (kernel, cc))
    return sym


def available(cc, kernel=None):
    """Tell if the kernels are present. With kernel=None, test all of them."""
    names = KERNELS if kernel is None else (kernel,)
    for name in names:
        try:
            library_path(name, cc)
        except (FileNotFoundError, KeyError):
            return False
    return True
