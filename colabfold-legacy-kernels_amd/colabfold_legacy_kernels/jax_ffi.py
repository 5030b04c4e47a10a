"""Registration of this package's XLA FFI targets with JAX on ROCm.

    from colabfold_legacy_kernels import jax_ffi
    jax_ffi.register()          # every target, platform "ROCM"

The reference leaves registration to its caller; the caller's code for the reference is
    jax.ffi.register_ffi_target(clk.symbol(k, cc), jax.ffi.pycapsule(getattr(lib, sym)),
                                platform="CUDA")
for each kernel k. This helper does the same for gfx950 with platform "ROCM", for the
reference's targets (VoltaMma, VoltaWmma, VoltaLayerNorm, VoltaGdp, VoltaGdpWmma) and for the
targets the reference lacks (the backward passes, fused LayerNorm + projections, the gate, the
pair bias, the triangle multiplication). jax is imported only when register() runs.
"""

import ctypes

from . import KERNELS, library_path, symbol

__all__ = ["targets", "register"]

# Targets exported beside the locator's symbol() names: the reference's sm_70 entry points.
_ALIASES = ("VoltaWmma", "VoltaGdpWmma")


def targets(cc="gfx950"):
    """[(target name, library path)] of every FFI target this package exports for ``cc``."""
    out = []
    for kernel in KERNELS:
        out.append((symbol(kernel, cc), library_path(kernel, cc)))
    lib_path = library_path("attention", cc)
    out += [(alias, lib_path) for alias in _ALIASES]
    seen, uniq = set(), []
    for name, path in out:
        if name not in seen:
            seen.add(name)
            uniq.append((name, path))
    return uniq


def register(platform="ROCM", cc="gfx950"):
    """Register every target with jax.ffi; returns the registered names."""
    try:
        import jax
    except ImportError as e:
        raise ImportError("colabfold_legacy_kernels.jax_ffi.register needs jax "
                          "(a ROCm build of jaxlib)") from e
    libs = {}
    names = []
    for name, path in targets(cc):
        lib = libs.get(path)
        if lib is None:
            lib = libs[path] = ctypes.CDLL(path)
        jax.ffi.register_ffi_target(name, jax.ffi.pycapsule(getattr(lib, name)),
                                    platform=platform)
        names.append(name)
    return names
