"""dscq_matmul_noalloc (include/dscq.h) through the C ABI: the GEMM whose K split
keeps its partial sums in the library's fixed device array instead of a
workspace.  Its outputs must equal dscq_matmul_ws's (the existing entry point,
with a torch-allocated workspace) bit for bit, on consecutive calls whose
second input is smaller -- the fixed array keeps the first call's contents --
and on a shape that does not split.  Every case is also checked against the
oracle's integer product.
"""
import numpy as np
import pytest
import torch

from dscquant_amd import _lib, w4a4
from oracle import native

pytestmark = pytest.mark.gpu


def _operands(M, N, K, seed, gpu):
    rng = np.random.default_rng(seed)
    MP, NP, KP = (M + 7) // 8 * 8, (N + 7) // 8 * 8, (K + 63) // 64 * 64
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    return dict(
        a=T(rng.integers(0, 256, size=(MP, KP // 2), dtype=np.uint8)),
        b=T(rng.integers(0, 256, size=(NP, KP // 2), dtype=np.uint8)),
        sx=T((rng.random(MP).astype(np.float32) + 0.5) * 0.05),
        zx=T(rng.integers(0, 16, size=MP).astype(np.int32)),
        sw=T((rng.random(NP).astype(np.float32) + 0.5) * 0.002),
        sums=T(rng.integers(-2000, 2000, size=NP).astype(np.int32)),
        bias=T((rng.standard_normal(N) * 0.1).astype(np.float16)),
        KP=KP)


def _call(name, o, M, N, gpu, extra=()):
    out = torch.empty((M, N), dtype=torch.float16, device=gpu)
    raw = torch.empty((M, N), dtype=torch.int32, device=gpu)
    _lib.call(name, o["a"].data_ptr(), o["b"].data_ptr(), o["sx"].data_ptr(),
              o["zx"].data_ptr(), o["sw"].data_ptr(), o["sums"].data_ptr(),
              o["bias"].data_ptr(), M, N, o["KP"], 0, 0, 0, out.data_ptr(), raw.data_ptr(),
              *extra, _lib.stream(gpu))
    return out, raw


@pytest.mark.parametrize("shapes", [[(128, 4096, 11008), (64, 4096, 11008), (2048, 4096, 4096)],
                                    [(32, 11008, 11008), (24, 4096, 8192)]])
def test_noalloc_matches_workspace_entry_point(gpu, shapes):
    for i, (M, N, K) in enumerate(shapes):
        print(f"matmul_noalloc call {i}: M{M} N{N} K{K}", flush=True)
        o = _operands(M, N, K, seed=M + N + K, gpu=gpu)
        need = w4a4.workspace_bytes(M, N, o["KP"])
        assert need <= _lib_scratch_bytes()
        ws = torch.empty((max(need, 16),), dtype=torch.uint8, device=gpu)
        out_ref, raw_ref = _call("dscq_matmul_ws", o, M, N, gpu, (ws.data_ptr(), need))
        out, raw = _call("dscq_matmul_noalloc", o, M, N, gpu)
        torch.cuda.synchronize()
        assert torch.equal(raw, raw_ref) and torch.equal(out, out_ref)
        if M * N * o["KP"] <= 6e9:
            a, b = o["a"].cpu().numpy(), o["b"].cpu().numpy()
            rows = np.arange(0, M, max(1, M // 16))
            cols = np.arange(0, N, max(1, N // 64))
            ia = native.unpack_int4(a[rows], o["KP"]).astype(np.int64)
            ib = native.unpack_int4(b[cols], o["KP"]).astype(np.int64)
            np.testing.assert_array_equal(raw.cpu().numpy()[np.ix_(rows, cols)], ia @ ib.T)


def _lib_scratch_bytes():
    import re
    import os
    text = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                             "include", "dscq.h")).read()
    m = re.search(r"#define DSCQ_NOALLOC_SCRATCH_BYTES \((\d+)LL << (\d+)\)", text)
    return int(m.group(1)) << int(m.group(2))
