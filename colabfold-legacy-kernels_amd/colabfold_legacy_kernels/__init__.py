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
    "attention_gate_bwd": ((_ARCH, _LIB, "ClkAttentionGateBwd"),),
    "attention_gated": ((_ARCH, _LIB, "ClkAttentionGated"),),
    "attention_nshd": ((_ARCH, _LIB, "ClkAttentionNshd"),),
    "attention_bwd_nshd": ((_ARCH, _LIB, "ClkAttentionBwdNshd"),),
    "ln_pair_bias": ((_ARCH, _LIB, "ClkLnPairBias"),),
    "gated_dual_proj_bwd": ((_ARCH, _LIB, "ClkGdpBwd"),),
    "triangle_multiply": ((_ARCH, _LIB, "ClkTriangleMultiply"),),
}

KERNELS = tuple(_TABLE)


def supported_capabilities():
    """Architectures with libraries in this package: only gfx950."""
    return _CAPABILITIES


def _normalise(cc):
    """``"gfx950"``, ``950`` and ``"950"`` name gfx950; any other number stays a number."""
    if isinstance(cc, str) and cc.strip().lower().startswith("gfx"):
        return cc.strip().lower()
    cc = int(cc)
    return _ARCH if cc == 950 else cc


def _resolve(kernel, cc):
    """(architecture, library file name or None, FFI target or None) for ``kernel`` on ``cc``.

    An unknown kernel name is a KeyError (the reference's message); an architecture this
    package was not built for resolves to no library and no target.
    """
    entries = _TABLE.get(kernel)
    if entries is None:
        raise KeyError(
            "unknown kernel %r, expected one of %s" % (kernel, ", ".join(KERNELS)))
    arch = _normalise(cc)
    match = next((e for e in entries if arch in _CAPABILITIES and e[0] == arch), None)
    return (arch, None, None) if match is None else (arch, match[1], match[2])


def _dirname(cc):
    return cc if isinstance(cc, str) else "sm%d" % cc


def _missing(kernel, arch):
    return FileNotFoundError("no %s kernel for architecture %s" % (kernel, arch))


def kernel_dir(cc):
    """Directory that holds (or would hold) the libraries built for ``cc``."""
    arch = _resolve("attention", cc)[0]
    return str(_KERNEL_DIR / _dirname(arch))


def library_path(kernel, cc):
    """Absolute path of the shared library with ``kernel`` for ``cc``.

    FileNotFoundError when the architecture has no build of it, or the file is absent.
    """
    arch, lib, _ = _resolve(kernel, cc)
    if lib is None:
        raise _missing(kernel, arch)
    path = _KERNEL_DIR / _dirname(arch) / lib
    if path.is_file():
        return str(path)
    raise FileNotFoundError("%s is not in this package" % path)


def symbol(kernel, cc):
    """Name of the XLA FFI handler symbol for ``kernel`` exported by its library."""
    arch, _, target = _resolve(kernel, cc)
    if target is None:
        raise _missing(kernel, arch)
    return target


def _present(kernel, cc):
    try:
        library_path(kernel, cc)
    except (FileNotFoundError, KeyError):
        return False
    return True


def available(cc, kernel=None):
    """True when ``kernel`` (every kernel, if None) has its library on disk for ``cc``."""
    return all(_present(name, cc) for name in (KERNELS if kernel is None else (kernel,)))
