"""The built library's gfx950 machine code: every matrix kernel issues MFMA instructions.

This is the counterpart of the reference's tensor-core check of its own build
(scripts/build_kernels.sh:120-150), applied to the AMD assembly of the library built here: the
device code objects are unbundled from the in-tree .so with llvm-objdump --offloading and
disassembled, and each kernel function is inspected on its own. A build that silently lost its
MFMA path (a wrong target, a fallback) fails here. It also checks that no packed-FP32 VALU form
was emitted: the build disables them for all device code.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

import colabfold_legacy_kernels as clk

OBJDUMP = Path("/opt/rocm/llvm/bin/llvm-objdump")

pytestmark = [
    pytest.mark.skipif(not clk.available("gfx950"), reason="library not built"),
    pytest.mark.skipif(not OBJDUMP.is_file(), reason="llvm-objdump not installed"),
]

# Kernel families that contract on the matrix cores (substring of the mangled name).
MFMA_KERNELS = ["attn_fwd_kernel", "attn_bwd_dq2", "attn_bwd_dkv2", "attn_bwd_dq",
                "attn_bwd_dkv", "gdp_kernel", "gdp_stream_kernel", "ln_gdp_kernel",
                "attn_gate_kernel", "tri_einsum_kernel", "tri_out_kernel",
                "gdp_bwd_grad_kernel", "gdp_bwd_dx_kernel", "gdp_bwd_dw_kernel"]
FUNC = re.compile(r"^[0-9a-f]+ <(?P<name>[^>]+)>:$")


@pytest.fixture(scope="module")
def functions(tmp_path_factory):
    """{mangled kernel name: [instruction mnemonics]} over every gfx950 code object."""
    work = tmp_path_factory.mktemp("objs")
    lib = work / "lib.so"
    shutil.copy(clk.library_path("attention", "gfx950"), lib)
    subprocess.run([str(OBJDUMP), "--offloading", str(lib)], check=True, cwd=work,
                   capture_output=True)
    objs = sorted(p for p in work.iterdir() if "amdgcn-amd-amdhsa--gfx950" in p.name)
    assert objs, "no gfx950 code object in the library"
    funcs = {}
    for obj in objs:
        text = subprocess.run([str(OBJDUMP), "-d", str(obj)], check=True, capture_output=True,
                              text=True).stdout
        cur = None
        for line in text.splitlines():
            m = FUNC.match(line.strip())
            if m:
                cur = funcs.setdefault(m.group("name"), [])
                continue
            if cur is not None:
                parts = line.strip().split()
                if parts and re.match(r"^[a-z_][a-z0-9_]*$", parts[0]):
                    cur.append(parts[0])
    return funcs


@pytest.mark.parametrize("family", MFMA_KERNELS)
def test_matrix_kernels_issue_mfma(functions, family):
    inst = {n: ops for n, ops in functions.items()
            if re.search(r"\d" + family + r"I", n) or n.endswith(family)}
    assert inst, "no instance of %s in the library" % family
    for name, ops in inst.items():
        n = sum(1 for o in ops if o.startswith("v_mfma"))
        assert n > 0, "%s has no MFMA instruction" % name


def test_attention_kernels_use_the_lds_transpose_read(functions):
    """The P.V and dQ products read V^T / K^T with ds_read_b64_tr_b16 (gfx950)."""
    for family in ("attn_fwd_kernel", "attn_bwd_dq2", "attn_bwd_dkv2"):
        inst = [ops for n, ops in functions.items() if family in n]
        assert inst and all(any(o.startswith("ds_read_b64_tr_b16") for o in ops)
                            for ops in inst), family


def test_no_packed_fp32_valu(functions):
    packed = {"v_pk_fma_f32", "v_pk_mul_f32", "v_pk_add_f32"}
    bad = sorted(n for n, ops in functions.items() if packed & set(ops))
    assert not bad, "packed FP32 VALU forms in: %s" % bad[:5]
