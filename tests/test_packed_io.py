"""On-disk packed-weight format (dscquant_amd.packed_io).

CPU: a layer packed by the oracle survives save -> load bit for bit, with its
metadata; malformed shapes and foreign files are refused.  GPU: weights packed
on the device, saved and reloaded, give the same GEMM output as before.
"""
import numpy as np
import pytest
import torch

from dscquant_amd import packed_io
from oracle import native
from tests.conftest import weights


def _oracle_pack(N, K, rot, seed=1):
    pw, sw, sums = native.pack_weight(weights(N, K, seed=seed).astype(np.float32), 1.0, rot)
    return torch.from_numpy(pw), torch.from_numpy(sw), torch.from_numpy(sums)


@pytest.mark.parametrize("N,K,rot,bias", [(100, 200, 0, False), (64, 256, 128, True)])
def test_round_trip(tmp_path, N, K, rot, bias):
    pw, sw, sums = _oracle_pack(N, K, rot)
    b = torch.randn(N).half() if bias else None
    path = str(tmp_path / "layer.safetensors")
    packed_io.save_packed(path, pw, sw, sums, K, N, rotate_block=rot, weight_clip=0.9, bias=b)
    got = packed_io.load_packed(path)
    assert torch.equal(got["packed"], pw) and torch.equal(got["sw"], sw)
    assert torch.equal(got["sums"], sums)
    assert (got["bias"] is None) == (b is None) and (b is None or torch.equal(got["bias"], b))
    assert (got["K"], got["N"], got["rotate_block"]) == (K, N, rot)
    assert got["weight_clip"] == 0.9
    # padded rows (N .. NP) carry scale 0 and sum 0
    assert not sw[N:].any() and not sums[N:].any()


def test_rejects_bad_shapes_and_files(tmp_path):
    pw, sw, sums = _oracle_pack(16, 128, 0)
    with pytest.raises(ValueError, match="packed must be uint8"):
        packed_io.save_packed(str(tmp_path / "a"), pw[:, :10], sw, sums, 128, 16)
    with pytest.raises(ValueError, match="sw must be"):
        packed_io.save_packed(str(tmp_path / "a"), pw, sw[:8], sums, 128, 16)
    with pytest.raises(ValueError, match="rotate_block"):
        packed_io.save_packed(str(tmp_path / "a"), pw, sw, sums, 128, 16, rotate_block=64)
    from safetensors.torch import save_file
    other = str(tmp_path / "other.safetensors")
    save_file({"packed": pw}, other, metadata={"format": "something-else"})
    with pytest.raises(ValueError, match="not a dscq-w4-packed/1 file"):
        packed_io.load_packed(other)


@pytest.mark.gpu
def test_reloaded_weights_give_the_same_output(gpu, tmp_path):
    from dscquant_amd import w4a4
    M, N, K = 40, 264, 512
    w = torch.from_numpy(weights(N, K, seed=4)).to(gpu)
    pw, sw, sums = w4a4.pack_weight(w, 1.0, 128)
    path = str(tmp_path / "w.safetensors")
    packed_io.save_packed(path, pw, sw, sums, K, N, rotate_block=128)
    got = packed_io.load_packed(path, device=gpu)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(3)).half().to(gpu)
    pa, sx, zx = w4a4.quantize(x, 1.0, True, got["rotate_block"])
    bias = torch.empty(0, dtype=torch.float16, device=gpu)
    y1, _ = w4a4.matmul(pa, pw, sx, zx, sw, sums, bias, M, N)
    y2, _ = w4a4.matmul(pa, got["packed"], sx, zx, got["sw"], got["sums"], bias, M, N)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
