"""Build the gfx950 kernel library in-tree.

    python colabfold-legacy-kernels_amd/build.py [--jobs N] [--asm]

Compiles every ``csrc/*.hip`` and ``csrc/*.cpp`` with hipcc for gfx950 into ``_build/`` and
links them into ``colabfold_legacy_kernels/kernels/gfx950/libclk_gfx950.so``, the file the
locator's ``library_path`` names. This is the counterpart of the reference's per-arch build
(scripts/build_kernels.sh:86-116): one target architecture, no CUTLASS, no XLA headers needed.

``--asm`` also writes the gfx950 assembly of each kernel source to ``_build/<name>.s`` (device
code only), for reading. The machine-code check itself -- the analogue of the reference's
tensor-core SASS check (scripts/build_kernels.sh:120-150) -- is ``tests/test_build.py``: it
unbundles the gfx950 code objects of the built library, disassembles them and asserts that every
matrix kernel issues ``v_mfma`` instructions.
"""

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
OUT_DIR = HERE / "colabfold_legacy_kernels" / "kernels" / "gfx950"
LIB = OUT_DIR / "libclk_gfx950.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 VALU forms are disabled for all device code: hipcc -O3 would otherwise form
# v_pk_{add,mul,fma}_f32 from scalar float code. MFMA results are allocated to ordinary VGPRs
# (not AGPRs): the kernels post-process every accumulator with VALU ops, which cannot read
# AGPRs, so the AGPR form costs a v_accvgpr_read per element and often an extra wave of
# register pressure.
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "--offload-arch=" + ARCH,
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-I" + str(REPO / "include"), "-I" + str(CSRC),
]


# Device-only flags of single sources. The attention forward's device code is compiled assuming
# no NaN operands: its running maxima then need no quieting of each operand before v_max (the
# scores are MFMA and FMA results, never signalling NaNs), about 12 VALU instructions fewer per
# 64-key tile. Host code keeps full NaN semantics (its argument checks test for NaN).
DEVICE_FLAGS = {"attention_fwd.hip": ["-Xarch_device", "-fno-honor-nans"]}


def sources():
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("command failed: %s\n%s%s" % (" ".join(cmd), res.stdout, res.stderr))
    return res


def _compile(src):
    obj = BUILD / (src.stem + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    _run([HIPCC] + COMMON + DEVICE_FLAGS.get(src.name, []) + lang +
         ["-c", str(src), "-o", str(obj)])
    return obj


def _asm(src):
    out = BUILD / (src.stem + ".s")
    _run([HIPCC] + COMMON + DEVICE_FLAGS.get(src.name, []) +
         ["-x", "hip", "--cuda-device-only", "-S", str(src), "-o", str(out)])
    return out


def check_ffi_layout(verbose=True):
    """Static-assert csrc/xla_ffi_abi.h against XLA's c_api.h when FFI_INCLUDE names it."""
    inc = os.environ.get("FFI_INCLUDE", "")
    if not inc or not (Path(inc) / "xla" / "ffi" / "api" / "c_api.h").is_file():
        if verbose:
            print("ffi layout check skipped (FFI_INCLUDE does not hold xla/ffi/api/c_api.h)")
        return False
    _run([HIPCC, "-std=c++17", "-fsyntax-only", "-I" + inc, "-I" + str(CSRC),
          str(CSRC / "xla_ffi_layout_check.cc")])
    if verbose:
        print("ffi layout check passed against", inc)
    return True


def build(jobs=None, asm=False, verbose=True):
    """Compile and link; returns the library path."""
    BUILD.mkdir(exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
        if asm:
            list(pool.map(_asm, [s for s in srcs if s.suffix == ".hip"]))
    tmp = LIB.with_name(LIB.name + ".tmp")
    # libstdc++ and libgcc linked statically (as the reference's build does,
    # scripts/build_kernels.sh:78-84): the library then needs only libc, libm, the loader and the
    # HIP runtime at load time (tests/test_packaging.py audits that).
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-static-libstdc++",
          "-static-libgcc", "-o", str(tmp)] + [str(o) for o in objs])
    os.replace(tmp, LIB)
    if verbose:
        print("built %s (%d units)" % (LIB, len(objs)))
    check_ffi_layout(verbose)
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--asm", action="store_true")
    args = ap.parse_args(argv)
    build(args.jobs, args.asm)
    return 0


if __name__ == "__main__":
    sys.exit(main())
