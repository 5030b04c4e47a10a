"""XLA FFI handlers driven by a fake XLA runtime (tests/_xla_ffi.py) on the CPU: the metadata
query, non-execute stages, and every decode/validation error path (no kernel is launched).
tests/test_gpu_ffi.py runs the same handlers on device buffers."""
import ctypes

import pytest

import colabfold_legacy_kernels as clk
from _xla_ffi import BF16, F16, F32, F64, S32, S64, U8, FakeXla, Metadata, MetadataExtension, \
    ExtensionBase, ApiVersion

pytestmark = pytest.mark.skipif(not clk.available("gfx950"), reason="library not built")

TARGETS = ["VoltaMma", "VoltaWmma", "ClkAttentionFwd", "ClkAttentionBwd", "VoltaLayerNorm",
           "ClkLayerNormBwd", "VoltaGdp", "VoltaGdpWmma", "ClkLnGdp", "ClkAttentionGate",
           "ClkAttentionGated", "ClkAttentionNshd", "ClkAttentionBwdNshd", "ClkLnPairBias",
           "ClkGdpBwd", "ClkTriangleMultiply", "ClkAttentionGateBwd"]
FAKE = 0x100000


@pytest.fixture
def lib():
    return ctypes.CDLL(clk.library_path("attention", "gfx950"))


@pytest.mark.parametrize("name", TARGETS)
def test_metadata_query(lib, name):
    x = FakeXla()
    md = Metadata(ctypes.sizeof(Metadata), ApiVersion(), 0)
    ext = MetadataExtension(ExtensionBase(ctypes.sizeof(MetadataExtension), 1, None),
                            ctypes.pointer(md))
    fr = x.frame([], [], extension=ext)
    assert x.call(lib, name, fr) is None
    assert (md.api_version.major_version, md.api_version.minor_version) == (0, 1)
    assert md.traits == 1  # command-buffer compatible
    assert x.errors == []


@pytest.mark.parametrize("name", TARGETS)
def test_non_execute_stages_do_nothing(lib, name):
    x = FakeXla()
    for stage in (0, 1, 2):
        assert x.call(lib, name, x.frame([], [], stage=stage)) is None
    assert x.errors == []


def attention_frame(x, n=2, h=2, sq=16, sk=16, d=32, dt=BF16, mask_dt=U8, bias_shape=None,
                    out_dt=None, attrs=None):
    args = [x.buffer(dt, (n, h, sq, d), FAKE), x.buffer(dt, (n, h, sk, d), FAKE),
            x.buffer(dt, (n, h, sk, d), FAKE), x.buffer(dt, bias_shape or (h, sq, sk), FAKE),
            x.buffer(mask_dt, (n, sk), FAKE)]
    rets = [x.buffer(out_dt or dt, (n, h, sq, d), FAKE)]
    if attrs is None:
        attrs = [("block_k", S64, 64), ("block_q", S64, 64), ("scale", F32, 0.17)]
    return x.frame(args, rets, attrs)


@pytest.mark.parametrize("kw,msg", [
    (dict(d=24), "head dim"), (dict(dt=F32), "f16 or all bf16"),
    (dict(mask_dt=BF16), "kmask"), (dict(bias_shape=(2, 16, 8)), "bias"),
    (dict(out_dt=F16), "result"), (dict(attrs=[("scale", F32, 0.1)]), "block_q"),
    (dict(attrs=[("block_q", S32, 64), ("block_k", S32, 64)]), "scale"),
])
def test_volta_mma_rejects(lib, kw, msg):
    x = FakeXla()
    err = x.call(lib, "VoltaMma", attention_frame(x, **kw))
    assert err is not None
    code, text = x.errors[-1]
    assert code == 3 and msg in text, text


def test_attention_attribute_types(lib):
    """f64 scale and i32 block sizes are accepted (decode), then the fake addresses fail the
    alignment-free empty-batch path: N = 0 returns OK without a launch."""
    x = FakeXla()
    fr = attention_frame(x, n=0, attrs=[("scale", F64, 0.17), ("block_q", S32, 32),
                                        ("block_k", S32, 32)])
    assert x.call(lib, "VoltaMma", fr) is None, x.errors


def test_layer_norm_rejects(lib):
    x = FakeXla()
    fr = x.frame([x.buffer(BF16, (4, 128), FAKE), x.buffer(BF16, (128,), FAKE),
                  x.buffer(F32, (128,), FAKE)], [x.buffer(BF16, (4, 128), FAKE)],
                 [("eps", F32, 1e-5)])
    assert x.call(lib, "VoltaLayerNorm", fr) is not None
    assert "scale and offset must be f32" in x.errors[-1][1]
    fr = x.frame([x.buffer(BF16, (4, 128), FAKE), x.buffer(F32, (128,), FAKE),
                  x.buffer(F32, (128,), FAKE)], [x.buffer(BF16, (4, 128), FAKE)], [])
    assert x.call(lib, "VoltaLayerNorm", fr) is not None
    assert "eps" in x.errors[-1][1]


def test_gdp_rejects_n_not_multiple_of_8(lib):
    x = FakeXla()
    m, k, n = 4, 128, 12
    fr = x.frame([x.buffer(BF16, (m, k), FAKE), x.buffer(BF16, (k, n), FAKE),
                  x.buffer(BF16, (n,), FAKE), x.buffer(BF16, (k, n), FAKE),
                  x.buffer(BF16, (n,), FAKE), x.buffer(BF16, (m,), FAKE)],
                 [x.buffer(BF16, (m, n), FAKE)])
    assert x.call(lib, "VoltaGdp", fr) is not None
    assert x.errors[-1][0] == 3 and "multiple of 8" in x.errors[-1][1]


def test_attention_bwd_rejects_small_workspace(lib):
    x = FakeXla()
    n, h, s, d = 2, 2, 16, 32
    q = lambda: x.buffer(BF16, (n, h, s, d), FAKE)  # noqa: E731
    args = [q(), q(), q(), x.buffer(BF16, (h, s, s), FAKE), x.buffer(U8, (n, s), FAKE), q(), q(),
            x.buffer(F32, (n, h, s), FAKE)]
    rets = [q(), q(), q(), x.buffer(F32, (h, s, s), FAKE), x.buffer(U8, (1,), FAKE)]
    assert x.call(lib, "ClkAttentionBwd", x.frame(args, rets, [("scale", F32, 0.17)])) is not None
    assert "workspace" in x.errors[-1][1]


def test_attention_bwd_nshd_decode_errors(lib):
    """ClkAttentionBwdNshd checks q, k, v, out, dout and the gradients in [N,S,H,D]."""
    x = FakeXla()
    n, h, sq, sk, d = 2, 4, 16, 24, 32
    qs = lambda: x.buffer(BF16, (n, sq, h, d), FAKE)  # noqa: E731
    ks = lambda: x.buffer(BF16, (n, sk, h, d), FAKE)  # noqa: E731
    args = [qs(), ks(), ks(), x.buffer(BF16, (h, sq, sk), FAKE), x.buffer(U8, (n, sk), FAKE),
            qs(), qs(), x.buffer(F32, (n, h, sq), FAKE)]
    rets = [qs(), ks(), ks(), x.buffer(F32, (h, sq, sk), FAKE), x.buffer(U8, (1,), FAKE)]
    scale = [("scale", F32, 0.17)]
    assert x.call(lib, "ClkAttentionBwdNshd", x.frame(args, rets, scale)) is not None
    assert "workspace" in x.errors[-1][1]  # every shape accepted, the 1-byte workspace is not
    bad_out = args[:5] + [x.buffer(BF16, (n, h, sq, d), FAKE)] + args[6:]
    assert x.call(lib, "ClkAttentionBwdNshd", x.frame(bad_out, rets, scale)) is not None
    assert "[N,Sq,H,D]" in x.errors[-1][1]
    bad_dk = rets[:1] + [x.buffer(BF16, (n, h, sk, d), FAKE)] + rets[2:]
    assert x.call(lib, "ClkAttentionBwdNshd", x.frame(args, bad_dk, scale)) is not None
    assert "dq, dk, dv" in x.errors[-1][1]
    # The [N,H,S,D] target rejects the same operands.
    assert x.call(lib, "ClkAttentionBwd", x.frame(args, rets, scale)) is not None
    assert "[N,H," in x.errors[-1][1]


def test_ln_gdp_operand_count(lib):
    x = FakeXla()
    fr = x.frame([x.buffer(BF16, (4, 128), FAKE)], [x.buffer(BF16, (4, 128), FAKE)],
                 [("eps", F32, 1e-5)])
    assert x.call(lib, "ClkLnGdp", fr) is not None
    assert "12 operands" in x.errors[-1][1]


def test_attention_gate_decode_errors(lib):
    x = FakeXla()
    fr = x.frame([x.buffer(BF16, (2, 8, 16, 32), FAKE), x.buffer(BF16, (2, 16, 256), FAKE),
                  x.buffer(BF16, (256, 128), FAKE), x.buffer(BF16, (256,), FAKE)],
                 [x.buffer(BF16, (2, 16, 256), FAKE)], [])
    assert x.call(lib, "ClkAttentionGate", fr) is not None
    assert "wg [C,H*D]" in x.errors[-1][1]
    fr = x.frame([x.buffer(BF16, (2, 8, 16, 32), FAKE)], [x.buffer(BF16, (2, 16, 256), FAKE)], [])
    assert x.call(lib, "ClkAttentionGate", fr) is not None
    assert "4 operands" in x.errors[-1][1]


def test_attention_gate_bwd_decode_errors(lib):
    x = FakeXla()
    ins = [x.buffer(BF16, (2, 8, 16, 32), FAKE), x.buffer(BF16, (2, 16, 256), FAKE),
           x.buffer(BF16, (256, 256), FAKE), x.buffer(BF16, (256,), FAKE),
           x.buffer(BF16, (2, 16, 256), FAKE)]
    outs = [x.buffer(BF16, (2, 8, 16, 32), FAKE), x.buffer(BF16, (2, 16, 256), FAKE),
            x.buffer(F32, (256, 256), FAKE), x.buffer(F32, (256,), FAKE),
            x.buffer(U8, (1 << 20,), FAKE)]
    fr = x.frame(ins[:4], outs, [])
    assert x.call(lib, "ClkAttentionGateBwd", fr) is not None
    assert "5 operands" in x.errors[-1][1]
    fr = x.frame(ins[:4] + [x.buffer(BF16, (2, 16, 128), FAKE)], outs, [])
    assert x.call(lib, "ClkAttentionGateBwd", fr) is not None
    assert "dout [N,Sq,H*D]" in x.errors[-1][1]
    fr = x.frame(ins, [x.buffer(BF16, (2, 16, 256), FAKE)] + outs[1:], [])
    assert x.call(lib, "ClkAttentionGateBwd", fr) is not None
    assert "do [N,H,Sq,D]" in x.errors[-1][1]
    fr = x.frame(ins, outs[:2] + [x.buffer(BF16, (256, 256), FAKE)] + outs[3:], [])
    assert x.call(lib, "ClkAttentionGateBwd", fr) is not None
    assert "dwg f32" in x.errors[-1][1]
    fr = x.frame(ins, outs[:4] + [x.buffer(F32, (1 << 18,), FAKE)], [])
    assert x.call(lib, "ClkAttentionGateBwd", fr) is not None
    assert "u8 workspace" in x.errors[-1][1]
    fr = x.frame(ins, outs[:4] + [x.buffer(U8, (64,), FAKE)], [])
    assert x.call(lib, "ClkAttentionGateBwd", fr) is not None
    assert "workspace" in x.errors[-1][1]


def test_attention_gated_decode_errors(lib):
    x = FakeXla()
    attn = [x.buffer(BF16, (2, 8, 16, 32), FAKE)] * 3 + [x.buffer(BF16, (8, 16, 16), FAKE),
                                                          x.buffer(U8, (2, 16), FAKE)]
    gate = [x.buffer(BF16, (2, 16, 128), FAKE), x.buffer(BF16, (128, 256), FAKE),
            x.buffer(BF16, (256,), FAKE)]
    res = [x.buffer(BF16, (2, 16, 256), FAKE)]
    scale = [("scale", F32, 0.17)]
    fr = x.frame(attn + gate[:2] + [x.buffer(BF16, (128,), FAKE)], res, scale)
    assert x.call(lib, "ClkAttentionGated", fr) is not None
    assert "bg [H*D]" in x.errors[-1][1]
    fr = x.frame(attn + gate, [x.buffer(BF16, (2, 8, 16, 32), FAKE)], scale)
    assert x.call(lib, "ClkAttentionGated", fr) is not None
    assert "result [N,Sq,H*D]" in x.errors[-1][1]
    fr = x.frame(attn + gate, res, [])
    assert x.call(lib, "ClkAttentionGated", fr) is not None
    assert "scale" in x.errors[-1][1]
    fr = x.frame(attn, res, scale)
    assert x.call(lib, "ClkAttentionGated", fr) is not None
    assert "8 operands" in x.errors[-1][1]
    fr = x.frame(attn + [x.buffer(BF16, (2, 16, 48), FAKE), x.buffer(BF16, (48, 256), FAKE),
                         gate[2]], res, scale)
    assert x.call(lib, "ClkAttentionGated", fr) is not None
    assert "multiple of 32" in x.errors[-1][1]


def test_new_targets_decode_errors(lib):
    x = FakeXla()
    fr = x.frame([x.buffer(BF16, (8, 8, 128), FAKE)], [x.buffer(BF16, (8, 8, 128), FAKE)], [])
    assert x.call(lib, "ClkTriangleMultiply", fr) is not None
    assert "18 operands" in x.errors[-1][1]
    fr = x.frame([x.buffer(BF16, (64, 128), FAKE)], [x.buffer(BF16, (64, 128), FAKE)], [])
    assert x.call(lib, "ClkGdpBwd", fr) is not None
    assert "7 operands" in x.errors[-1][1]
    fr = x.frame([x.buffer(BF16, (4, 4, 128), FAKE), x.buffer(F32, (128,), FAKE),
                  x.buffer(F32, (128,), FAKE), x.buffer(BF16, (128, 4), FAKE)],
                 [x.buffer(BF16, (4, 4, 4), FAKE)], [])
    assert x.call(lib, "ClkLnPairBias", fr) is not None
    assert "eps" in x.errors[-1][1]


@pytest.mark.parametrize("name", TARGETS)
def test_stream_get_failure_fails_the_call(lib, name):
    """When XLA cannot hand over the platform stream the handler returns XLA's own error and
    launches nothing (the frame's operands are fake addresses: a launch would fault)."""
    x = FakeXla(stream_error=True)
    fr = attention_frame(x) if "Attention" in name or name.startswith("VoltaMma") or \
        name == "VoltaWmma" else x.frame([], [])
    err = x.call(lib, name, fr)
    assert err == 0xE5
    assert x.stream_gets == 1 and x.errors == []


def test_attention_nshd_decode_errors(lib):
    """ClkAttentionNshd: q, k, v and the result in [N,S,H,D]; every shape and dtype checked on the
    host before the C ABI is called."""
    x = FakeXla()
    q = x.buffer(BF16, (2, 16, 8, 32), FAKE)      # [N, Sq, H, D]
    kv = x.buffer(BF16, (2, 24, 8, 32), FAKE)     # [N, Sk, H, D]
    bias, km = x.buffer(BF16, (8, 16, 24), FAKE), x.buffer(U8, (2, 24), FAKE)
    res = [x.buffer(BF16, (2, 16, 8, 32), FAKE)]
    scale = [("scale", F32, 0.17)]
    cases = [
        ([q, kv, kv, bias], res, scale, "5 operands"),
        ([q, x.buffer(BF16, (2, 24, 4, 32), FAKE), kv, bias, km], res, scale, "[N,Sk,H,D]"),
        ([q, kv, kv, x.buffer(BF16, (8, 24, 16), FAKE), km], res, scale, "bias"),
        ([q, kv, kv, bias, x.buffer(BF16, (2, 24), FAKE)], res, scale, "kmask"),
        ([q, kv, kv, bias, km], [x.buffer(BF16, (2, 8, 16, 32), FAKE)], scale, "result"),
        ([q, kv, kv, bias, km], res, [], "scale"),
        ([x.buffer(F32, (2, 16, 8, 32), FAKE), kv, kv, bias, km], res, scale, "f16 or all bf16"),
        ([x.buffer(BF16, (2, 16, 8, 24), FAKE), x.buffer(BF16, (2, 24, 8, 24), FAKE),
          x.buffer(BF16, (2, 24, 8, 24), FAKE), bias, km], [x.buffer(BF16, (2, 16, 8, 24), FAKE)],
         scale, "head dim"),
    ]
    for args, rets, attrs, msg in cases:
        assert x.call(lib, "ClkAttentionNshd", x.frame(args, rets, attrs)) is not None, msg
        assert msg in x.errors[-1][1], (msg, x.errors[-1][1])
