"""The C ABI from several host threads at once, each on its own stream (ctypes
releases the GIL, so the calls overlap): every thread's quantize -> matmul and
fused decode results equal the same calls made one after another, bit for bit.
"""
import threading

import numpy as np
import pytest
import torch

from dscquant_amd import w4a4
from tests.conftest import activations, weights

pytestmark = pytest.mark.gpu


def test_concurrent_threads_match_sequential(gpu):
    print("threads: 4 host threads x 20 iterations, own streams", flush=True)
    K, N = 4096, 4096
    pw, sw, sums = w4a4.pack_weight(torch.from_numpy(weights(N, K, seed=3)).to(gpu), 1.0, 128)
    bias = torch.empty(0, dtype=torch.float16, device=gpu)
    shapes = [1, 4, 16, 300]
    xs = {M: [torch.from_numpy(activations(M, K, seed=10 * M + i).astype(np.float16)).to(gpu)
              for i in range(4)] for M in shapes}

    def call(M, x):
        if M <= 4 and w4a4.linear_decode_supported(M, K):
            return w4a4.linear_decode(x, 1.0, 128, pw, sw, sums, bias, N)
        pa, sx, zx = w4a4.quantize(x, 1.0, True, 128)
        out, _ = w4a4.matmul(pa, pw, sx, zx, sw, sums, bias, M, N)
        return out

    ref = {M: [call(M, x).clone() for x in xs[M]] for M in shapes}
    torch.cuda.synchronize()
    errors = []

    def worker(M):
        try:
            stream = torch.cuda.Stream(device=gpu)
            with torch.cuda.stream(stream):
                for it in range(20):
                    i = it % len(xs[M])
                    y = call(M, xs[M][i])
                    stream.synchronize()
                    if not torch.equal(y, ref[M][i]):
                        errors.append((M, it))
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((M, repr(e)))

    ts = [threading.Thread(target=worker, args=(M,)) for M in shapes]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in ts), "a worker thread did not finish"
    assert errors == []
