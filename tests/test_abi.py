"""C-ABI and host-boundary tests that need no GPU.

* libdscq.so loads and exports every function declared in include/dscq.h;
* the C entry points reject bad arguments before touching the GPU, with the
  reference extension's messages (kernel/w4a4.cu:165-168, 197);
* the Python wrappers reproduce the reference's RuntimeError / ValueError
  messages (kernel/w4a4.cu:12-17, 192-202; core/quantization.py:32-36);
* the product path refuses CPU tensors instead of falling back.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import dscquant_amd
from dscquant_amd import _lib, w4a4
from dscquant_amd.core import quantization as Q
from dscquant_amd.core.linear import QuantLinear

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dscq.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dscq_\w+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    L = _lib.lib()
    names = header_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(L, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with dscq.h"


def test_version_and_no_gpu_here():
    L = _lib.lib()
    assert L.dscq_version().startswith(b"dscq ")
    if not torch.cuda.is_available():
        assert L.dscq_device_supported() <= 0


def _einval(name, *args):
    L = _lib.lib()
    rc = getattr(L, name)(*args)
    assert rc == -1
    return L.dscq_last_error().decode()


def test_c_quantize_argument_checks():
    # (x, dtype, M, K, clip, fused, rotate, packed, scales, zeros, codes, stream)
    dummy = 16
    assert _einval("dscq_quantize", dummy, 7, 1, 64, 1.0, 1, 0, dummy, dummy, dummy, None,
                   None) == "Only FP16 and FP32 inputs are supported"
    for M, K in ((0, 64), (65536, 64), (1, 0), (1, 1048577)):
        assert _einval("dscq_quantize", dummy, 0, M, K, 1.0, 1, 0, dummy, dummy, dummy, None,
                       None) == "Require 1<=M<=65535 and 1<=K<=1048576"
    for clip in (0.49, 1.01):
        assert _einval("dscq_quantize", dummy, 0, 4, 64, clip, 1, 0, dummy, dummy, dummy, None,
                       None) == "Activation clip must be in [0.5,1]"
    assert "multiple of 128" in _einval("dscq_quantize", dummy, 0, 4, 192, 1.0, 1, 128, dummy,
                                        dummy, dummy, None, None)
    assert "rotate_block" in _einval("dscq_quantize", dummy, 0, 4, 256, 1.0, 1, 64, dummy,
                                     dummy, dummy, None, None)
    assert "codes buffer" in _einval("dscq_quantize", dummy, 0, 4, 64, 1.0, 0, 0, dummy, dummy,
                                     dummy, None, None)


def test_c_matmul_argument_checks():
    d = 16
    for M, N, KP in ((0, 8, 64), (65536, 8, 64), (4, 0, 64), (4, 8, 96), (4, 8, 0),
                     (4, 8, 1048576 + 64)):
        assert _einval("dscq_matmul", d, d, d, d, d, d, None, M, N, KP, 1, 0, 0, d, None,
                       None) == "Invalid dimensions"
    assert "raw buffer" in _einval("dscq_matmul", d, d, d, d, d, d, None, 4, 8, 64, 0, 0, 0, d,
                                   None, None)


def test_c_matmul_ws_argument_checks_and_workspace_query():
    d = 16
    for M, N, KP in ((0, 8, 64), (65536, 8, 64), (4, 8, 96)):
        assert _einval("dscq_matmul_ws", d, d, d, d, d, d, None, M, N, KP, 1, 0, 0, d, None,
                       None, 0, None) == "Invalid dimensions"
        assert _lib.lib().dscq_matmul_workspace_bytes(M, N, KP, 0) < 0
    assert "workspace" in _einval("dscq_matmul_ws", d, d, d, d, d, d, None, 4, 8, 64, 1, 0, 0,
                                  d, None, None, -1, None)
    q = _lib.lib().dscq_matmul_workspace_bytes
    # host-only: few 64 x 128 tiles with a long K split into int32 parts of
    # [M, N] (256 compute units assumed where no device is visible)
    assert q(128, 4096, 11008, 0) == 4 * 128 * 4096 * 4
    assert q(512, 4096, 11008, 0) == 0      # the tiles already fill the CUs
    assert q(128, 4096, 4096, 0) == 0       # K too short to pay for the second pass
    assert q(2048, 4096, 4096, 0) == 0      # full rounds of 256 x 128 tiles
    assert q(8, 4096, 4096, 0) == 0         # skinny-M kernel
    assert q(128, 4096, 4096, 1) == 0       # forced decode
    assert q(512, 4100, 11008, 0) == 0      # N % 8 != 0: general kernel
    assert w4a4.workspace_bytes(128, 4096, 11008) == 4 * 128 * 4096 * 4


def test_c_matmul_noalloc_argument_checks():
    d = 16
    for M, N, KP in ((0, 8, 64), (65536, 8, 64), (4, 0, 64), (4, 8, 96)):
        assert _einval("dscq_matmul_noalloc", d, d, d, d, d, d, None, M, N, KP, 1, 0, 0, d,
                       None, None) == "Invalid dimensions"
    assert "raw buffer" in _einval("dscq_matmul_noalloc", d, d, d, d, d, d, None, 4, 8, 64, 0,
                                   0, 0, d, None, None)
    assert "null buffer" in _einval("dscq_matmul_noalloc", None, d, d, d, d, d, None, 4, 8, 64,
                                    1, 0, 0, d, None, None)


def test_c_other_argument_checks():
    d = 16
    assert "bits" in _einval("dscq_activation_codes", d, 0, 4, 64, 1.0, 9, 0, d, d, d, None)
    assert "clip" in _einval("dscq_activation_codes", d, 0, 4, 64, 0.0, 4, 0, d, d, d, None)
    assert "Weight clip" in _einval("dscq_pack_weight", d, 0, 4, 64, 1.5, 0, d, d, d, None, None)
    assert "bits" in _einval("dscq_weight_codes", d, 0, 4, 64, 1.0, 1, 0, d, d, None)
    assert "width" in _einval("dscq_unpack_int4", d, 2, 3, 7, d, None)
    assert "N<=32768" in _einval("dscq_silu_mul_quantize", d, d, 40000, 4, 40000, 1.0, 0, d, d,
                                 d, None, None)
    assert "stride" in _einval("dscq_silu_mul_quantize", d, d, 8, 4, 16, 1.0, 0, d, d, d, None,
                               None)
    assert "multiple of 128" in _einval("dscq_silu_mul_quantize", d, d, 384, 4, 192, 1.0, 128,
                                        d, d, d, None, None)


def test_c_set_gemm_kernel_is_per_thread():
    import threading
    L = _lib.lib()
    assert L.dscq_set_gemm_kernel(1) == 0
    seen = []
    t = threading.Thread(target=lambda: seen.append(L.dscq_set_gemm_kernel(0)))
    t.start()
    t.join()
    assert seen == [0]  # a new thread starts at automatic
    assert L.dscq_set_gemm_kernel(0) == 1
    assert "0 to 4" in _einval("dscq_set_gemm_kernel", 5)


def test_c_probe_argument_checks():
    d = 16
    assert "pieces" in _einval("dscq_stream_probe", d, 64, d, 16, 3, None)
    assert "multiple" in _einval("dscq_stream_probe", d, 48, d, 0, 4, None)
    assert "write_bytes" in _einval("dscq_stream_probe", d, 256, d, 32, 4, None)
    assert "aligned" in _einval("dscq_stream_probe", 8, 256, d, 64, 4, None)
    assert "waves" in _einval("dscq_mfma_probe", 4, 9, 64, d, None)
    assert "multiple of 8" in _einval("dscq_mfma_probe", 4, 8, 12, d, None)
    assert "workgroups" in _einval("dscq_mfma_probe", 0, 8, 64, d, None)


def test_c_linear_decode_limits_and_checks():
    L = _lib.lib()
    # One 128-element block per quad of a 512-lane workgroup: M * ceil(KP/128) <= 128.
    assert L.dscq_linear_decode_supported(1, 4096) == 1
    assert L.dscq_linear_decode_supported(4, 4096) == 1
    assert L.dscq_linear_decode_supported(5, 4096) == 0
    assert L.dscq_linear_decode_supported(2, 8192) == 1
    assert L.dscq_linear_decode_supported(1, 11008) == 1
    assert L.dscq_linear_decode_supported(2, 11008) == 0
    assert L.dscq_linear_decode_supported(1, 16384) == 0   # weight stripe > 12 blocks/wave
    assert L.dscq_linear_decode_supported(1, 4100) == 0    # K % 8
    assert L.dscq_linear_decode_supported(0, 64) == 0
    d = 16
    # (x, dtype, M, K, clip, rotate, b, sw, sums, bias, N, fp32, out, stream)
    assert "exceed" in _einval("dscq_linear_decode", d, 0, 5, 4096, 1.0, 0, d, d, d, None, 8,
                               0, d, None)
    assert _einval("dscq_linear_decode", d, 3, 1, 64, 1.0, 0, d, d, d, None, 8, 0, d,
                   None) == "Only FP16 and FP32 inputs are supported"
    assert _einval("dscq_linear_decode", d, 0, 1, 64, 1.0, 0, d, d, d, None, 0, 0, d,
                   None) == "Invalid dimensions"
    assert "clip" in _einval("dscq_linear_decode", d, 0, 1, 64, 0.2, 0, d, d, d, None, 8, 0, d,
                             None)
    assert "multiple of 128" in _einval("dscq_linear_decode", d, 0, 1, 192, 1.0, 128, d, d, d,
                                        None, 8, 0, d, None)
    assert "null" in _einval("dscq_linear_decode", d, 0, 1, 64, 1.0, 0, None, d, d, None, 8, 0,
                             d, None)
    assert "aligned" in _einval("dscq_linear_decode", 8, 0, 1, 64, 1.0, 0, d, d, d, None, 8, 0,
                                d, None)


# ------------------------------------------------------- Python-side messages

def test_quantize_messages_match_reference():
    x = torch.zeros(4, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="Expected contiguous CUDA tensor"):
        w4a4.quantize(x, 1.0, True)
    chk = w4a4.check_quantize_args
    with pytest.raises(RuntimeError, match="Only FP16 and FP32 inputs are supported"):
        chk(x.to(torch.bfloat16), 1.0, require_cuda=False)
    with pytest.raises(RuntimeError, match=r"Require 1<=M<=65535 and 1<=K<=1048576"):
        chk(torch.zeros(65536, 1, dtype=torch.float16), 1.0, require_cuda=False)
    with pytest.raises(RuntimeError, match=r"Require 1<=M<=65535"):
        chk(torch.zeros(4, 64, 2, dtype=torch.float16), 1.0, require_cuda=False)
    with pytest.raises(RuntimeError, match=r"Activation clip must be in \[0.5,1\]"):
        chk(x, 0.25, require_cuda=False)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        chk(torch.zeros(4, 64, dtype=torch.float16), 1.0, 128, require_cuda=False)
    chk(x, 0.5, require_cuda=False)


def _mm_args(M=4, N=16, KP=64, fp32=False):
    MP, NP = (M + 7) // 8 * 8, (N + 7) // 8 * 8
    a = torch.zeros(MP, KP // 2, dtype=torch.uint8)
    b = torch.zeros(NP, KP // 2, dtype=torch.uint8)
    sx = torch.zeros(MP)
    zx = torch.zeros(MP, dtype=torch.int32)
    sw = torch.zeros(NP)
    sums = torch.zeros(NP, dtype=torch.int32)
    bias = torch.zeros(0, dtype=torch.float32 if fp32 else torch.float16)
    return dict(a=a, b=b, sx=sx, zx=zx, sw=sw, sums=sums, bias=bias, M=M, N=N, fp32=fp32)


def test_matmul_messages_match_reference():
    chk = lambda **k: w4a4.check_matmul_args(require_cuda=False, **k)  # noqa: E731
    assert chk(**_mm_args()) == 64
    with pytest.raises(RuntimeError, match="Expected contiguous CUDA tensor"):
        w4a4.matmul(*_mm_args().values())
    bad = _mm_args(); bad["a"] = bad["a"].to(torch.int8)
    with pytest.raises(RuntimeError, match="Packed operands must be byte matrices"):
        chk(**bad)
    bad = _mm_args(); bad["a"] = torch.zeros(8, 48, dtype=torch.uint8); bad["b"] = torch.zeros(16, 48, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="Invalid dimensions"):
        chk(**bad)
    bad = _mm_args(); bad["M"] = 0
    with pytest.raises(RuntimeError, match="Invalid dimensions"):
        chk(**bad)
    bad = _mm_args(M=9)
    bad["a"] = torch.zeros(8, 32, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="Invalid padded operand shapes"):
        chk(**bad)
    bad = _mm_args(); bad["b"] = torch.zeros(16, 64, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="Invalid padded operand shapes"):
        chk(**bad)
    bad = _mm_args(); bad["zx"] = bad["zx"].float()
    with pytest.raises(RuntimeError, match="Invalid metadata dtypes"):
        chk(**bad)
    bad = _mm_args(); bad["sw"] = torch.zeros(8)
    with pytest.raises(RuntimeError, match="Metadata too short"):
        chk(**bad)
    bad = _mm_args(); bad["bias"] = torch.zeros(16)
    with pytest.raises(RuntimeError, match="Bias shape/dtype mismatch"):
        chk(**bad)
    bad = _mm_args(fp32=True); bad["bias"] = torch.zeros(15)
    with pytest.raises(RuntimeError, match="Bias shape/dtype mismatch"):
        chk(**bad)


def test_pack_int4_messages_match_reference():
    with pytest.raises(ValueError, match="Packed weights must be a matrix."):
        Q.pack_int4(torch.zeros(3, dtype=torch.int8))
    with pytest.raises(ValueError, match="Signed INT4 code out of range."):
        Q.pack_int4(torch.tensor([[8, 0]]))
    with pytest.raises(ValueError, match="Signed INT4 code out of range."):
        Q.pack_int4(torch.tensor([[-9, 0]]))


def test_no_cpu_fallback():
    x = torch.randn(4, 64)
    with pytest.raises(RuntimeError, match="runs on the GPU"):
        Q.activation_codes(x, 4)
    with pytest.raises(RuntimeError, match="runs on the GPU"):
        Q.weight_codes(x, 4)
    with pytest.raises(RuntimeError, match="runs on the GPU"):
        Q.pack_int4(torch.zeros(2, 2, dtype=torch.int8))
    with pytest.raises(RuntimeError, match="runs on the GPU"):
        Q.unpack_int4(torch.zeros(2, 2, dtype=torch.uint8), 4)


def test_quant_linear_keeps_reference_state_and_defaults():
    class Cfg:
        weight_bits = 4
        activation_bits = 4

    base = torch.nn.Linear(64, 32)
    ql = QuantLinear(base, Cfg())
    assert ql.enabled is False
    keys = set(ql.state_dict())
    assert keys == {"weight_clip", "activation_clip", "base.weight", "base.bias"}
    assert not any(p.requires_grad for p in base.parameters())
    x = torch.randn(3, 64)
    torch.testing.assert_close(ql(x), base(x))  # disabled: plain base forward
    ql.enabled = True
    with pytest.raises(RuntimeError):
        ql(x)  # enabled on a CPU tensor: no silent fallback


def test_transformed_fold_rules():
    """core/linear.py:22-46 fold rules with duck-typed Rotation / Scaling objects."""
    torch.manual_seed(0)

    class Rot(torch.nn.Module):
        def __init__(self, heads, head_dim):
            super().__init__()
            self.heads, self.head_dim = heads, head_dim
            q, _ = torch.linalg.qr(torch.randn(heads, head_dim, head_dim))
            self.m = q

        def matrices(self):
            return self.m

    class Scl(torch.nn.Module):
        def __init__(self, n):
            super().__init__()
            self.s = torch.rand(n) + 0.5

        def diagonal(self):
            return self.s

    cfg = type("C", (), {"weight_bits": 4, "activation_bits": 4})()
    rot = Rot(2, 8)
    base_v = torch.nn.Linear(32, 16)
    w, b = QuantLinear(base_v, cfg, rot, "v").transformed()
    R = rot.m
    torch.testing.assert_close(w, (R.transpose(-1, -2) @ base_v.weight.reshape(2, 8, 32)).reshape(16, 32))
    torch.testing.assert_close(b, (R.transpose(-1, -2) @ base_v.bias.reshape(2, 8, 1)).flatten())
    base_o = torch.nn.Linear(16, 32)
    w, _ = QuantLinear(base_o, cfg, rot, "o").transformed()
    ref = torch.einsum("ohd,hde->ohe", base_o.weight.reshape(32, 2, 8), R).reshape(32, 16)
    torch.testing.assert_close(w, ref)
    scl = Scl(16)
    base_up = torch.nn.Linear(8, 16)
    w, b = QuantLinear(base_up, cfg, scl, "up").transformed()
    torch.testing.assert_close(w, base_up.weight / scl.s[:, None])
    torch.testing.assert_close(b, base_up.bias / scl.s)
    base_dn = torch.nn.Linear(16, 8)
    w, _ = QuantLinear(base_dn, cfg, scl, "down").transformed()
    torch.testing.assert_close(w, base_dn.weight * scl.s[None, :])


def test_interleave_gate_up_order():
    """Rows of gate and up interleaved in 64-row blocks (the gated GEMM's weight order)."""
    import torch
    from dscquant_amd import w4a4
    N = 192
    gate = torch.arange(N, dtype=torch.int32)
    up = torch.arange(N, dtype=torch.int32) + 1000
    il = w4a4.interleave_gate_up(gate, up)
    expect = []
    for t in range(N // 64):
        expect += list(range(64 * t, 64 * t + 64)) + list(range(1000 + 64 * t, 1000 + 64 * t + 64))
    assert il.tolist() == expect
    g2, u2 = gate.reshape(N, 1).repeat(1, 3), up.reshape(N, 1).repeat(1, 3)
    assert torch.equal(w4a4.interleave_gate_up(g2, u2)[:, 0], il)
    with pytest.raises(RuntimeError):
        w4a4.interleave_gate_up(gate[:100], up[:100])


def test_last_error_is_per_thread():
    """dscq_last_error() reports the calling thread's own last failure: two
    threads failing with different messages, interleaved, each read theirs."""
    import threading
    L = _lib.lib()
    dummy = 16
    barrier = threading.Barrier(2, timeout=10)
    seen = {}

    def worker(name, dtype, M, want):
        msgs = []
        for _ in range(200):
            rc = L.dscq_quantize(dummy, dtype, M, 64, 1.0, 1, 0, dummy, dummy, dummy, None, None)
            assert rc == -1
            barrier.wait()
            msgs.append(L.dscq_last_error().decode())
            barrier.wait()
        seen[name] = set(msgs)
        assert seen[name] == {want}

    ts = [threading.Thread(target=worker, args=("a", 7, 4, "Only FP16 and FP32 inputs are supported")),
          threading.Thread(target=worker, args=("b", 0, 0, "Require 1<=M<=65535 and 1<=K<=1048576"))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert seen == {"a": {"Only FP16 and FP32 inputs are supported"},
                    "b": {"Require 1<=M<=65535 and 1<=K<=1048576"}}
