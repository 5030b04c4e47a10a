"""Packaging on the CPU, mirroring the reference's release checks
(.github/workflows/build-and-publish.yml:54-90):

* the library's dynamic dependencies are only the C library, libm, the loader and the HIP
  runtime (libstdc++ and libgcc are linked statically, scripts/build_kernels.sh:78-84);
* a wheel built from colabfold-legacy-kernels_amd/ installs and its locator finds every
  library and FFI symbol (the reference's wheel smoke test, with gfx950 for sm_70/75);
* the JAX registration helper registers every target with platform "ROCM" (against a stand-in
  for jax, which is not installed here).
"""
import ctypes
import os
import shutil
import subprocess
import sys
import types
from pathlib import Path

import pytest

import colabfold_legacy_kernels as clk

ROOT = Path(__file__).resolve().parents[1]
PKG_ROOT = ROOT / "colabfold-legacy-kernels_amd"

pytestmark = pytest.mark.skipif(not clk.available("gfx950"), reason="library not built")

ALLOWED = ("libamdhip64.so", "libc.so", "libm.so", "ld-linux-x86-64.so")


def needed(path):
    out = subprocess.run(["readelf", "-d", path], check=True, capture_output=True,
                         text=True).stdout
    return [line.split("[", 1)[1].rstrip("]").strip() for line in out.splitlines()
            if "(NEEDED)" in line]


@pytest.mark.skipif(shutil.which("readelf") is None, reason="readelf not installed")
def test_library_links_only_libc_and_the_hip_runtime():
    path = clk.library_path("attention", "gfx950")
    deps = needed(path)
    assert deps, "no dynamic section"
    bad = [d for d in deps if not d.startswith(ALLOWED)]
    assert not bad, "unexpected dynamic dependencies: %s" % bad
    assert not any(d.startswith(("libstdc++", "libgcc_s")) for d in deps)
    if shutil.which("ldd"):
        out = subprocess.run(["ldd", path], capture_output=True, text=True).stdout
        assert "not found" not in out, out


SMOKE = r"""
import ctypes
import colabfold_legacy_kernels as clk
assert clk.__file__.startswith(SITE), clk.__file__
assert clk.available("gfx950"), "gfx950 reports unavailable"
for kernel in clk.KERNELS:
    path = clk.library_path(kernel, "gfx950")
    assert path.startswith(SITE), path
    lib = ctypes.cdll.LoadLibrary(path)
    getattr(lib, clk.symbol(kernel, "gfx950"))
for cc in (70, 75, 80):
    assert not clk.available(cc)
print("smoke test OK")
"""


@pytest.mark.skipif(shutil.which("pip") is None and shutil.which("pip3") is None,
                    reason="pip not installed")
def test_wheel_installs_and_locates_every_target(tmp_path):
    env = dict(os.environ, CLK_SKIP_KERNEL_BUILD="1")
    dist, site = tmp_path / "dist", tmp_path / "site"
    subprocess.run([sys.executable, "-m", "pip", "wheel", "--no-deps", "--no-build-isolation",
                    "-q", "-w", str(dist), str(PKG_ROOT)], check=True, env=env,
                   capture_output=True)
    wheels = list(dist.glob("colabfold_legacy_kernels-*.whl"))
    assert len(wheels) == 1, wheels
    assert "-py3-none-linux_x86_64" in wheels[0].name, wheels[0].name
    subprocess.run([sys.executable, "-m", "pip", "install", "--no-deps", "-q", "--target",
                    str(site), str(wheels[0])], check=True, capture_output=True)
    assert (site / "colabfold_legacy_kernels" / "kernels" / "gfx950" /
            "libclk_gfx950.so").is_file()
    out = subprocess.run([sys.executable, "-c", "SITE = %r\n" % str(site) + SMOKE],
                         cwd=tmp_path, env=dict(os.environ, PYTHONPATH=str(site)),
                         capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    assert "smoke test OK" in out.stdout


def test_jax_registration_helper(monkeypatch):
    from colabfold_legacy_kernels import jax_ffi
    calls = []
    fake = types.ModuleType("jax")
    fake.ffi = types.SimpleNamespace(
        pycapsule=lambda fn: ("capsule", ctypes.cast(fn, ctypes.c_void_p).value),
        register_ffi_target=lambda name, cap, platform: calls.append((name, cap, platform)))
    monkeypatch.setitem(sys.modules, "jax", fake)
    names = jax_ffi.register()
    expected = {clk.symbol(k, "gfx950") for k in clk.KERNELS} | {"VoltaWmma", "VoltaGdpWmma"}
    assert set(names) == expected and len(names) == len(expected)
    assert all(platform == "ROCM" for _, _, platform in calls)
    assert all(cap[0] == "capsule" and cap[1] for _, cap, _ in calls)


def test_jax_registration_needs_jax(monkeypatch):
    from colabfold_legacy_kernels import jax_ffi
    monkeypatch.setitem(sys.modules, "jax", None)  # import jax raises ImportError
    with pytest.raises(ImportError, match="needs jax"):
        jax_ffi.register()
