"""The C ABI library on the CPU: it loads, exports every symbol include/clk.h declares and every
XLA FFI target the locator names, and rejects invalid calls before any GPU work. No kernel runs
here (this machine may have no GPU): every call below fails host-side validation."""
import ctypes
import re
from pathlib import Path

import pytest

import colabfold_legacy_kernels as clk
from colabfold_legacy_kernels import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "clk.h"

pytestmark = pytest.mark.skipif(not clk.available("gfx950"),
                                reason="library not built (run __graft_entry__.build())")


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(clk_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(clk.library_path("attention", "gfx950"))
    names = declared_functions()
    assert len(names) >= 12, names
    for name in names:
        getattr(lib, name)
    assert set(names) == set(_native.PROTOTYPES), "ctypes prototypes out of sync with clk.h"


def test_every_ffi_target_is_exported():
    for kernel in clk.KERNELS:
        lib = ctypes.CDLL(clk.library_path(kernel, "gfx950"))
        getattr(lib, clk.symbol(kernel, "gfx950"))
    lib = ctypes.CDLL(clk.library_path("attention", "gfx950"))
    for alias in ("VoltaWmma", "VoltaGdpWmma"):  # the reference's sm_70 target names
        getattr(lib, alias)


def test_version_and_last_error():
    lib = _native.lib()
    assert b"gfx950" in lib.clk_version()
    assert isinstance(lib.clk_last_error(), bytes)


def test_profile_hooks_without_launches():
    lib = _native.lib()
    lib.clk_profile_enable(1)
    lib.clk_profile_enable(0)
    assert _native.collect() == []


INVALID = _native.INVALID_ARGUMENT
BF16, F16, F32, U8 = _native.BF16, _native.F16, _native.F32, _native.U8
FAKE = 0x100000  # a non-null, 16-byte aligned address that is never dereferenced


def attn_fwd(**kw):
    a = dict(stream=None, dtype=BF16, q=FAKE, k=FAKE, v=FAKE, bias=FAKE, kmask=FAKE, out=FAKE,
             lse=None, N=2, H=2, Sq=16, Sk=16, D=32, scale=0.17, bq=64, bk=64)
    a.update(kw)
    return _native.lib().clk_attention_fwd(*a.values())


@pytest.mark.parametrize("kw,msg", [
    (dict(D=24), "head dim"), (dict(D=128), "head dim"), (dict(dtype=F32), "dtype"),
    (dict(dtype=U8), "dtype"), (dict(N=-1), "negative"), (dict(q=None), "null"),
    (dict(out=FAKE + 8), "aligned"), (dict(bq=0), "positive"), (dict(N=70000), "too large"),
])
def test_attention_fwd_validation(kw, msg):
    assert attn_fwd(**kw) == INVALID
    assert msg in _native.last_error()


def attn_fwd_nshd(**kw):
    a = dict(stream=None, dtype=BF16, q=FAKE, k=FAKE, v=FAKE, bias=FAKE, kmask=FAKE, out=FAKE,
             lse=None, N=2, H=2, Sq=16, Sk=16, D=32, scale=0.17)
    a.update(kw)
    return _native.lib().clk_attention_fwd_nshd(*a.values())


@pytest.mark.parametrize("kw,msg", [
    (dict(D=24), "head dim"), (dict(dtype=F32), "dtype"), (dict(N=-1), "negative"),
    (dict(q=None), "null"), (dict(v=FAKE + 8), "aligned"),
    # [N,S,H,D] rows of one (n, h) lie H*D apart: S*H*D*2 must fit 31 bits.
    (dict(H=4096, Sq=8192, Sk=8192, D=64), "[N,S,H,D]"),
])
def test_attention_fwd_nshd_validation(kw, msg):
    assert attn_fwd_nshd(**kw) == INVALID
    assert msg in _native.last_error()
    assert attn_fwd_nshd(N=0) == _native.OK


def test_attention_fwd_empty_is_ok():
    assert attn_fwd(N=0) == _native.OK
    assert attn_fwd(Sq=0) == _native.OK


def test_attention_bwd_validation():
    lib = _native.lib()
    ws = lib.clk_attention_bwd_workspace_size(384, 4, 384, 384, 32)
    assert ws > 384 * 4 * 384 * 4  # at least the D_i row sums
    args = [None, BF16] + [FAKE] * 5 + [FAKE, FAKE, FAKE] + [FAKE] * 4 + [FAKE, ws - 1,
                                                                         384, 4, 384, 384, 32, 0.17]
    assert lib.clk_attention_bwd(*args) == INVALID
    assert "workspace" in _native.last_error()
    args[-7] = ws
    args[-2] = 12
    assert lib.clk_attention_bwd(*args) == INVALID
    assert "head dim" in _native.last_error()


def test_attention_bwd_nshd_validation():
    lib = _native.lib()
    dims = [384, 4, 384, 384, 32]
    ws = lib.clk_attention_bwd_workspace_size(*dims)
    args = [None, BF16] + [FAKE] * 12 + [FAKE, ws - 1] + dims + [0.17]
    assert lib.clk_attention_bwd_nshd(*args) == INVALID
    assert "workspace" in _native.last_error()
    args[15] = ws
    args[-2] = 12
    assert lib.clk_attention_bwd_nshd(*args) == INVALID
    assert "head dim" in _native.last_error()
    # [N,S,H,D] rows of one (n, h) lie H*D apart: S*H*D*2 must fit 31 bits.
    big = [1, 4096, 8192, 8192, 64]
    args = [None, BF16] + [FAKE] * 12 + [FAKE, 1 << 40] + big + [0.17]
    assert lib.clk_attention_bwd_nshd(*args) == INVALID
    assert "[N,S,H,D]" in _native.last_error()


def test_attention_bwd_noalloc_refuses_sizes_beyond_its_scratch():
    """Host-side check before any device call: the 1024-residue problem needs more workspace
    than the fixed scratch array holds."""
    lib = _native.lib()
    limit = lib.clk_attention_bwd_noalloc_limit()
    assert limit == 64 << 20
    dims = (1024, 4, 1024, 1024, 32)
    assert lib.clk_attention_bwd_workspace_size(*dims) > limit
    assert lib.clk_attention_bwd_noalloc(None, BF16, *([FAKE] * 12), *dims, 0.17) == INVALID
    assert "scratch" in _native.last_error()
    assert lib.clk_attention_bwd_noalloc(None, BF16, *([FAKE] * 12), -1, 4, 8, 8, 32,
                                         0.17) == INVALID


def test_stream_copy_validation():
    lib = _native.lib()
    assert lib.clk_stream_copy(None, FAKE, FAKE, 0) == _native.OK
    assert lib.clk_stream_copy(None, FAKE, FAKE, 40) == INVALID       # not a multiple of 16
    assert lib.clk_stream_copy(None, FAKE + 8, FAKE, 64) == INVALID   # misaligned
    assert lib.clk_stream_copy(None, None, FAKE, 64) == INVALID


def test_issue_calibration_validation():
    lib = _native.lib()
    assert lib.clk_issue_calibration(None, 7, 256, 256, 10, FAKE) == INVALID   # no such kind
    assert lib.clk_issue_calibration(None, -1, 256, 256, 10, FAKE) == INVALID
    assert lib.clk_issue_calibration(None, 0, 0, 256, 10, FAKE) == INVALID     # no blocks
    assert lib.clk_issue_calibration(None, 0, 256, 96, 10, FAKE) == INVALID    # not whole waves
    assert lib.clk_issue_calibration(None, 0, 256, 2048, 10, FAKE) == INVALID  # too many threads
    assert lib.clk_issue_calibration(None, 0, 256, 256, 0, FAKE) == INVALID    # no rounds
    assert lib.clk_issue_calibration(None, 0, 256, 256, 10, None) == INVALID
    assert "issue_calibration" in _native.last_error()


def test_workspace_sizes_are_deterministic():
    lib = _native.lib()
    a = lib.clk_attention_bwd_workspace_size(384, 4, 384, 384, 32)
    assert a == lib.clk_attention_bwd_workspace_size(384, 4, 384, 384, 32)
    assert lib.clk_attention_bwd_workspace_size(-1, 4, 8, 8, 32) == 0
    assert lib.clk_layer_norm_bwd_workspace_size(512 * 512, 128) > 0
    assert lib.clk_layer_norm_bwd_workspace_size(0, 128) == 0


def test_layer_norm_validation():
    lib = _native.lib()
    assert lib.clk_layer_norm_fwd(None, U8, FAKE, FAKE, FAKE, FAKE, 4, 128, 1e-5) == INVALID
    assert lib.clk_layer_norm_fwd(None, BF16, FAKE, FAKE, FAKE, FAKE, 4, 0, 1e-5) == INVALID
    assert lib.clk_layer_norm_fwd(None, BF16, None, FAKE, FAKE, FAKE, 4, 128, 1e-5) == INVALID
    assert lib.clk_layer_norm_fwd(None, BF16, FAKE, FAKE, FAKE, FAKE, 0, 128, 1e-5) == _native.OK
    assert lib.clk_layer_norm_bwd(None, BF16, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 4, 128,
                                  1e-5) == INVALID


@pytest.mark.parametrize("m,k,n,msg", [(4, 128, 12, "multiple of 8"), (4, 12, 0, "bad dims"),
                                       (4, 0, 64, "bad dims"), (-1, 8, 8, "bad dims")])
def test_gdp_validation(m, k, n, msg):
    lib = _native.lib()
    assert lib.clk_gated_dual_proj(None, BF16, *([FAKE] * 7), m, k, n) == INVALID
    assert msg in _native.last_error()


@pytest.mark.parametrize("c,n", [(100, 128), (128, 160), (256, 128), (16, 32)])
def test_ln_gdp_validation(c, n):
    lib = _native.lib()
    assert lib.clk_ln_gated_dual_proj(None, BF16, *([FAKE] * 14), 4, c, n, 1e-5) == INVALID
    assert "multiples of 32" in _native.last_error()


@pytest.mark.parametrize("n,h,sq,d,c,msg", [(2, 8, 16, 32, 96, "64, 128 or 256"),
                                            (2, 3, 16, 32, 128, "64, 128 or 256"),
                                            (2, 4, 16, 12, 128, "multiple of 8"),
                                            (-1, 4, 16, 32, 128, "bad dims")])
def test_attention_gate_validation(n, h, sq, d, c, msg):
    lib = _native.lib()
    assert lib.clk_attention_gate(None, BF16, *([FAKE] * 5), n, h, sq, d, c) == INVALID
    assert msg in _native.last_error()


def gate_bwd(**kw):
    a = dict(stream=None, dtype=BF16, o=FAKE, x=FAKE, wg=FAKE, bg=FAKE, dout=FAKE, d_o=FAKE,
             dx=FAKE, dwg=FAKE, dbg=FAKE, workspace=FAKE, workspace_bytes=1 << 40, N=2, H=8,
             Sq=70, D=32, C=256, accumulate_dx=0)
    a.update(kw)
    return _native.lib().clk_attention_gate_bwd(*a.values())


@pytest.mark.parametrize("kw,msg", [
    (dict(dtype=F32), "dtype"), (dict(D=12, H=4), "multiple of 8"), (dict(H=0), "H > 0"),
    (dict(C=96), "64, 128 or 256"), (dict(H=3), "64, 128 or 256"),
    (dict(N=1 << 28, Sq=16), "too many"), (dict(Sq=1 << 21), "too long"),
    (dict(dwg=None), "null gradient"),
    (dict(o=None), "null operand"), (dict(workspace=None), "null operand"),
    (dict(d_o=FAKE + 8), "aligned"), (dict(wg=FAKE + 8), "aligned"),
    (dict(workspace_bytes=4096), "workspace"),
])
def test_attention_gate_bwd_validation(kw, msg):
    assert gate_bwd(**kw) == INVALID
    assert msg in _native.last_error()


def test_attention_gate_bwd_workspace_size():
    lib = _native.lib()
    ws = lib.clk_attention_gate_bwd_workspace_size(512, 8, 256, 32, 256)
    assert ws >= 512 * 256 * 256 * 2  # dg in the input dtype, then the partials
    assert ws == lib.clk_attention_gate_bwd_workspace_size(512, 8, 256, 32, 256)
    assert lib.clk_attention_gate_bwd_workspace_size(0, 8, 256, 32, 256) == 0


def attn_gated(**kw):
    a = dict(stream=None, dtype=BF16, q=FAKE, k=FAKE, v=FAKE, bias=FAKE, kmask=FAKE, x=FAKE,
             wg=FAKE, bg=FAKE, gated=FAKE, out=None, lse=None, N=2, H=2, Sq=16, Sk=16, D=32,
             C=64, scale=0.17)
    a.update(kw)
    return _native.lib().clk_attention_fwd_gated(*a.values())


@pytest.mark.parametrize("kw,msg", [
    (dict(C=48), "multiple of 32"), (dict(C=0), "multiple of 32"), (dict(D=24), "head dim"),
    (dict(dtype=F32), "dtype"), (dict(x=None), "null"), (dict(gated=None), "null"),
    (dict(wg=FAKE + 8), "aligned"), (dict(out=FAKE + 8), "aligned"),
    (dict(Sq=1 << 20, C=1024), "too large"), (dict(H=64, D=64, C=1 << 17), "too large"),
])
def test_attention_gated_validation(kw, msg):
    assert attn_gated(**kw) == INVALID
    assert msg in _native.last_error()


def test_attention_gated_empty_is_ok():
    assert attn_gated(N=0) == _native.OK
    assert attn_gated(Sq=0, x=None) == _native.OK  # no work: pointers are not needed


@pytest.mark.parametrize("m,k,n,msg", [(4, 96, 128, "64 or 128"), (4, 128, 32, "64 or 128"),
                                       (-1, 128, 128, "64 or 128"),
                                       (1 << 31, 128, 128, "too large")])
def test_gdp_bwd_validation(m, k, n, msg):
    lib = _native.lib()
    assert lib.clk_gated_dual_proj_bwd(None, BF16, *([FAKE] * 13), 1 << 30, m, k, n, 0) == INVALID
    assert msg in _native.last_error()


def tri_mul(**kw):
    arr = lambda n: (ctypes.c_void_p * n)(*([FAKE] * n))  # noqa: E731
    a = dict(stream=None, dtype=BF16, z=FAKE, mask=FAKE, ln=arr(4), w=arr(6), b=arr(6), out=FAKE,
             workspace=FAKE, workspace_bytes=1 << 62, N=64, C=128, outgoing=1, eps=1e-5)
    a.update(kw)
    return _native.lib().clk_triangle_multiply(*a.values())


@pytest.mark.parametrize("kw,msg", [
    (dict(C=96), "64 or 128"), (dict(dtype=F32), "dtype"), (dict(N=16385), "too large"),
    (dict(N=20000, C=64), "too large"), (dict(z=None), "null"), (dict(ln=None), "null"),
    (dict(out=FAKE + 8), "aligned"), (dict(workspace_bytes=1024), "workspace"),
])
def test_triangle_multiply_validation(kw, msg):
    assert tri_mul(**kw) == INVALID
    assert msg in _native.last_error()


def test_triangle_multiply_sizes():
    """The largest grid is accepted up to the workspace check; its workspace holds three
    channel-major plane sets of 2 bytes per element (ragged N adds the padded z, mask, out)."""
    lib = _native.lib()
    assert tri_mul(N=16384, workspace_bytes=1024) == INVALID
    assert "workspace" in _native.last_error()
    assert lib.clk_triangle_multiply_workspace_size(16384, 128) == 3 * 128 * 16384 ** 2 * 2
    assert lib.clk_triangle_multiply_workspace_size(4000, 64) == 3 * 64 * 4000 ** 2 * 2
    assert lib.clk_triangle_multiply_workspace_size(4001, 64) > 4 * 64 * 4008 ** 2 * 2
    assert tri_mul(N=0) == _native.OK
