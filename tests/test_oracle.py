"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is chosen so a plausible slip in the restatement (a dropped term,
a wrong rounding rule, a swapped nibble, a transposed operand, a wrong
butterfly sign) fails: closed-form special cases, exact .5 ties built on
power-of-two scales, range invariants, the exhaustive nibble table, the
integer GEMM against numpy's integer matmul, the transform against the dense
Sylvester matrix, and the fake-quant identity of the whole linear.
"""
import numpy as np
import pytest
import torch

from oracle import fakequant, native, numpy_ref
from tests.conftest import activations, weights


def f16(a):
    return np.asarray(a, dtype=np.float16).astype(np.float32)


# ----------------------------------------------------------------- activations

def test_activation_all_zero_row():
    codes, s, z = native.activation_codes(np.zeros((2, 64), np.float32))
    assert (codes == 0).all()
    assert (s == np.float32(1e-8)).all() and (z == 0).all()


def test_activation_all_positive_and_all_negative_rows():
    x = np.stack([np.linspace(0.5, 3.0, 64), -np.linspace(0.5, 3.0, 64)]).astype(np.float32)
    codes, s, z = native.activation_codes(x)
    assert z[0] == 0 and z[1] == 15            # lo = 0  /  hi = 0
    assert codes[0].max() == 15 and codes[1].min() == 0
    # all-positive: scale = max / 15 exactly as fp32 division
    assert s[0] == np.float32(np.float32(3.0) / np.float32(15))


def test_activation_constant_row():
    x = np.full((1, 32), 2.5, np.float32)
    codes, s, z = native.activation_codes(x)
    assert s[0] == np.float32(np.float32(2.5) / np.float32(15)) and z[0] == 0
    assert (codes == 15).all()


def test_activation_exact_ties_round_half_even():
    # lo = 0, hi = 15/8 -> scale = 1/8 exactly, zero = 0; x = (k + .5)/8 sits on
    # the tie k + .5, which must round to the even neighbour.
    ks = np.arange(15)
    row = np.concatenate([[0.0, 15 / 8], (ks + 0.5) / 8]).astype(np.float32)
    codes, s, z = native.activation_codes(row[None])
    assert s[0] == np.float32(0.125) and z[0] == 0
    expect = np.where(ks % 2 == 0, ks, ks + 1)
    assert codes[0, 0] == 0 and codes[0, 1] == 15
    np.testing.assert_array_equal(codes[0, 2:], expect)


def test_activation_zero_point_tie():
    # Build -lo/scale = 2.5 exactly with scale 1/8:
    # lo = -2.5/8, hi = 12.5/8 -> zero = rne(2.5) = 2 (even), not 3.
    row = np.array([[-2.5 / 8, 12.5 / 8, 0.0]], np.float32)
    codes, s, z = native.activation_codes(row)
    assert s[0] == np.float32(0.125)
    assert z[0] == 2
    # x = hi: 12.5 + 2 = 14.5 -> 14;  x = lo: -2.5 + 2 = -.5 -> -0 -> 0
    assert codes[0, 1] == 14 and codes[0, 0] == 0 and codes[0, 2] == 2


@pytest.mark.parametrize("clip", [1.0, 0.9, 0.5])
def test_activation_invariants(clip):
    x = f16(activations(64, 512, seed=3))
    codes, s, z = native.activation_codes(x, clip=clip)
    assert codes.max() <= 15
    mn, mx = x.min(axis=1), x.max(axis=1)
    assert (mn < 0).all() and (mx > 0).all()
    if clip == 1.0:
        # the row minimum maps to 0; the maximum to 15 (14 only on a .5 tie)
        assert (codes[np.arange(64), x.argmin(axis=1)] == 0).all()
        assert (codes[np.arange(64), x.argmax(axis=1)] >= 14).all()
    # scale / zero closed form
    lo = np.minimum(mn, 0).astype(np.float32) * np.float32(clip)
    hi = np.maximum(mx, 0).astype(np.float32) * np.float32(clip)
    np.testing.assert_array_equal(s, np.maximum((hi - lo) / np.float32(15), np.float32(1e-8)))
    # reconstruction error <= scale / 2 inside the clipped range
    deq = (codes.astype(np.float32) - z[:, None]) * s[:, None]
    inside = (x >= lo[:, None]) & (x <= hi[:, None])
    err = np.abs(deq - x)[inside] / np.broadcast_to(s[:, None], x.shape)[inside]
    assert err.max() <= 0.5 + 1e-5


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_activation_c_numpy_torch_agree(bits):
    x = f16(activations(16, 384, seed=bits))
    c1, s1, z1 = native.activation_codes(x, bits=bits, clip=0.75)
    c2, s2, z2 = numpy_ref.activation_codes(x, bits=bits, clip=0.75)
    c3, s3, z3 = fakequant.activation_codes(torch.from_numpy(x), bits, 0.75)
    np.testing.assert_array_equal(c1, c2)
    np.testing.assert_array_equal(c1, c3.numpy().astype(np.uint8))
    np.testing.assert_array_equal(s1, s3.numpy()[:, 0])
    np.testing.assert_array_equal(z1, z3.numpy()[:, 0])


# --------------------------------------------------------------------- weights

def test_weight_zero_row_and_reach():
    w = f16(weights(8, 256))
    w[3] = 0
    codes, s = native.weight_codes(w)
    assert (codes[3] == 0).all() and s[3] == np.float32(1e-8)
    live = np.arange(8) != 3
    assert (np.abs(codes[live]).max(axis=1) == 7).all()
    assert codes.min() >= -7 and codes.max() <= 7


def test_weight_exact_ties():
    # amax = 7/4 -> scale = 1/4 exactly; w = (k + .5)/4 ties to even.
    ks = np.arange(-6, 6)
    row = np.concatenate([[7 / 4], (ks + 0.5) / 4]).astype(np.float32)
    codes, s = native.weight_codes(row[None])
    assert s[0] == np.float32(0.25)
    r = ks + 0.5
    expect = np.where(np.floor(r) % 2 == 0, np.floor(r), np.ceil(r))
    np.testing.assert_array_equal(codes[0, 1:], expect.astype(np.int8))


@pytest.mark.parametrize("clip", [1.0, 0.6])
def test_weight_c_numpy_torch_agree(clip):
    w = f16(weights(32, 320, seed=5))
    c1, s1 = native.weight_codes(w, clip=clip)
    c2, s2 = numpy_ref.weight_codes(w, clip=clip)
    c3, s3 = fakequant.weight_codes(torch.from_numpy(w), 4, clip)
    np.testing.assert_array_equal(c1, c2)
    np.testing.assert_array_equal(c1, c3.numpy().astype(np.int8))
    np.testing.assert_array_equal(s1, s3.numpy()[:, 0])


# ----------------------------------------------------------------- int4 packing

def test_pack_table_exhaustive():
    c = np.array([[a, b] for a in range(-8, 8) for b in range(-8, 8)], np.int8)
    packed = native.pack_int4(c)
    expect = np.array([(a & 15) | ((b & 15) << 4) for a in range(-8, 8) for b in range(-8, 8)],
                      np.uint8)
    np.testing.assert_array_equal(packed[:, 0], expect)
    np.testing.assert_array_equal(native.unpack_int4(packed, 2), c)
    np.testing.assert_array_equal(numpy_ref.pack_int4(c), packed)
    np.testing.assert_array_equal(numpy_ref.unpack_int4(packed, 2), c)


def test_pack_odd_width_pads_zero():
    c = np.array([[1, -2, 3], [-8, 7, -1]], np.int8)
    p = native.pack_int4(c)
    assert p.shape == (2, 2)
    assert p[0, 1] == 3 and p[1, 1] == 15
    np.testing.assert_array_equal(native.unpack_int4(p, 3), c)


# -------------------------------------------------------------------- transform

def test_fwht_matches_dense_sylvester():
    x = f16(activations(8, 512, seed=7))
    y = native.fwht_rows(x, 128)
    H = numpy_ref.sylvester(128)
    dense = (x.reshape(8, 4, 128).astype(np.float64) @ H).reshape(8, 512)
    assert np.abs(y - dense).max() <= 1e-5 * np.abs(dense).max()
    np.testing.assert_array_equal(y, numpy_ref.fwht_rows(x, 128))


def test_fwht_exact_on_small_integers_and_involution():
    rng = np.random.default_rng(0)
    x = rng.integers(-100, 100, size=(4, 256)).astype(np.float32)
    H = numpy_ref.sylvester(128)
    y = native.fwht_rows(x, 128)
    np.testing.assert_array_equal(y, (x.reshape(4, 2, 128) @ H).reshape(4, 256))
    np.testing.assert_array_equal(native.fwht_rows(y, 128), 128 * x)  # H H = 128 I


def test_fwht_first_row_and_column_are_plain_sums():
    x = np.zeros((1, 128), np.float32)
    x[0, 5] = 1.0
    y = native.fwht_rows(x, 128)
    np.testing.assert_array_equal(np.abs(y), np.ones((1, 128), np.float32))
    assert y[0, 0] == 1.0  # H[0, :] is all +1


# ------------------------------------------------------------------ quantize_rows

def test_quantize_rows_padding():
    x = f16(activations(5, 100, seed=9))  # MP = 8, KP = 128
    packed, s, z, codes = native.quantize_rows(x, want_codes=True)
    assert packed.shape == (8, 64) and codes.shape == (8, 128)
    c_ref, s_ref, z_ref = native.activation_codes(x)
    np.testing.assert_array_equal(codes[:5, :100], c_ref)
    np.testing.assert_array_equal(s[:5], s_ref)
    np.testing.assert_array_equal(z[:5], z_ref.astype(np.int32))
    # padded k take the zero-point, padded rows are all 0x88 with scale 1e-8
    assert (codes[:5, 100:] == z[:5, None]).all()
    assert (packed[5:] == 0x88).all() and (s[5:] == np.float32(1e-8)).all() and (z[5:] == 0).all()
    # nibble = (q - 8) & 15, low nibble first
    q = codes.astype(np.int16)
    expect = (((q[:, 0::2] - 8) & 15) | (((q[:, 1::2] - 8) & 15) << 4)).astype(np.uint8)
    np.testing.assert_array_equal(packed, expect)


# ----------------------------------------------------------------- GEMM + restore

def test_gemm_raw_matches_integer_matmul():
    rng = np.random.default_rng(1)
    a = rng.integers(0, 256, size=(16, 96), dtype=np.uint8)   # every nibble value
    b = rng.integers(0, 256, size=(24, 96), dtype=np.uint8)
    raw = native.gemm_raw(a, b, 13, 21)
    ia = native.unpack_int4(a, 192).astype(np.int64)
    ib = native.unpack_int4(b, 192).astype(np.int64)
    np.testing.assert_array_equal(raw, (ia @ ib.T)[:13, :21])


def test_gemm_raw_extremes():
    a = np.full((8, 32), 0x88, np.uint8)  # every nibble -8
    b = np.full((8, 32), 0x88, np.uint8)
    raw = native.gemm_raw(a, b, 8, 8)
    assert (raw == 64 * 64).all()
    b2 = np.full((8, 32), 0x77, np.uint8)  # +7
    assert (native.gemm_raw(a, b2, 8, 8) == -56 * 64).all()


def test_restore_closed_form():
    rng = np.random.default_rng(2)
    M, N = 6, 10
    raw = rng.integers(-5000, 5000, size=(M, N)).astype(np.int32)
    sx = rng.random(M).astype(np.float32)
    zx = rng.integers(0, 16, size=M).astype(np.int32)
    sw = rng.random(N).astype(np.float32) * 0.01
    sums = rng.integers(-300, 300, size=N).astype(np.int32)
    bias = rng.standard_normal(N).astype(np.float32)
    out = native.restore(raw, sx, zx, sw, sums, bias, out_dtype=np.float32)
    exact = (raw + (8 - zx[:, None]) * sums[None, :]).astype(np.float64) * sx[:, None] * sw[None, :] + bias
    assert np.abs(out - exact).max() <= 1e-6 * np.abs(exact).max()
    # no bias, fp16 narrowing is round-to-nearest-even of the fp32 value
    o32 = native.restore(raw, sx, zx, sw, sums, None, out_dtype=np.float32)
    o16 = native.restore(raw, sx, zx, sw, sums, None)
    np.testing.assert_array_equal(o16, o32.astype(np.float16))


@pytest.mark.parametrize("rot", [0, 128])
def test_linear_identity_with_fake_quant(rot):
    """Integer path == F.linear(quantize_activation, quantize_weight) in exact arithmetic."""
    M, N, K = 8, 48, 256
    x = f16(activations(M, K, seed=11))
    w = f16(weights(N, K, seed=12))
    out, raw, (pa, sx, zx), (pw, sw, sums) = native.linear_w4a4(x, w, rotate_block=rot,
                                                                out_dtype=np.float32)
    xr = native.fwht_rows(x, rot) if rot else x
    wr = native.fwht_rows(w, rot) / np.float32(rot) if rot else w
    qa, s_a, z_a = numpy_ref.activation_codes(xr)
    cw, s_w = numpy_ref.weight_codes(wr)
    exact = ((qa.astype(np.float64) - z_a[:, None]) * s_a[:, None]) @ \
        (cw.astype(np.float64) * s_w[:, None]).T
    assert np.abs(out - exact).max() <= 2e-6 * np.abs(exact).max()
    # the fake-quant torch restatement on the same fp32 operands agrees to fp32
    fq = fakequant.forward(torch.from_numpy(xr), torch.from_numpy(wr), None).numpy()
    assert np.abs(out - fq).max() <= 1e-5 * np.abs(fq).max()


def test_linear_vs_fp16_fake_quant():
    """In fp16 the reference rounds x_hat and W_hat before F.linear: within ~1e-3."""
    M, N, K = 8, 48, 256
    x = activations(M, K, seed=11)
    w = weights(N, K, seed=12)
    out, *_ = native.linear_w4a4(f16(x), f16(w), out_dtype=np.float32)
    fq = fakequant.forward(torch.from_numpy(x).float(), torch.from_numpy(w).float(), None,
                           w_hat=fakequant.quantize_weight(torch.from_numpy(w).float(), 4)).numpy()
    fq16 = fakequant.forward(torch.from_numpy(x), torch.from_numpy(w), None).float().numpy()
    assert np.abs(out - fq).max() <= 1e-3 * np.abs(fq).max()
    assert np.abs(out - fq16).max() <= 5e-3 * np.abs(fq16).max()


def test_rotation_preserves_the_product():
    """(W H/128)(H x) = W x: the rotated path approximates the plain product."""
    M, N, K = 16, 64, 512
    x = f16(activations(M, K, seed=13))
    w = f16(weights(N, K, seed=14))
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    xr = native.fwht_rows(x, 128).astype(np.float64)
    wr = native.fwht_rows(w, 128).astype(np.float64) / 128
    np.testing.assert_allclose(xr @ wr.T, exact, rtol=1e-5, atol=1e-5)
    out_r, *_ = native.linear_w4a4(x, w, rotate_block=128, out_dtype=np.float32)
    out_p, *_ = native.linear_w4a4(x, w, rotate_block=0, out_dtype=np.float32)
    # with outlier channels, rotating first must cut the quantization error
    assert np.abs(out_r - exact).mean() < np.abs(out_p - exact).mean()


def test_pack_weight_matches_components():
    w = f16(weights(20, 200, seed=15))   # NP = 24, KP = 256
    packed, sw, sums = native.pack_weight(w, clip=0.9)
    codes, s = native.weight_codes(w, clip=0.9)
    np.testing.assert_array_equal(sw[:20], s)
    assert (sw[20:] == 0).all() and (sums[20:] == 0).all()
    np.testing.assert_array_equal(sums[:20], codes.astype(np.int64).sum(axis=1))
    np.testing.assert_array_equal(native.unpack_int4(packed, 256)[:20, :200], codes)
    assert (native.unpack_int4(packed, 256)[:20, 200:] == 0).all()
    assert (packed[20:] == 0).all()


def test_gemm_raw_blas_equals_brute_force():
    rng = np.random.default_rng(4)
    a = rng.integers(0, 256, size=(40, 160), dtype=np.uint8)
    b = rng.integers(0, 256, size=(56, 160), dtype=np.uint8)
    np.testing.assert_array_equal(native.gemm_raw_blas(a, b, 37, 50), native.gemm_raw(a, b, 37, 50))
