"""The fp8-activation kernels: the device row quantiser (bf16 rows -> OCP
e4m3 codes + one scale per row) against the library's host quantiser (the
one the e4m3 weights go through), bit for bit; and the fp8 x fp8 GEMM
(v_mfma_f32_16x16x128_f8f6f4) against fp64 products of the decoded codes,
through mfh_debug_quantize_rows_e4m3 and mfh_debug_gemm_fp8."""

import numpy as np
import pytest

from metalfish_amd import backend

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if backend.device_count() < 1:
        pytest.fail("GPU tests need an MI355X; none visible")


def _bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _f(b):
    return (np.asarray(b).astype(np.uint32) << 16).view(np.float32)


def _decode_e4m3(codes):
    """OCP e4m3 (bias 7, subnormals m * 2^-9, 0x7F / 0xFF NaN) as float64."""
    c = np.asarray(codes).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return sign * val


@pytest.mark.parametrize("rows,cols,split", [(64, 1024, True), (37, 1536, False),
                                             (8, 256, True), (5, 2048, True)])
def test_row_quantiser_matches_host(rows, cols, split):
    rng = np.random.default_rng(rows * cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[:, :7] *= 1e-3  # small values: e4m3 subnormal codes after scaling
    x[1 % rows] = 0.0  # a zero row: scale 1
    hi = _bits(x)
    lo = _bits(x - _f(hi)) if split else None
    xf = _f(hi) + (_f(lo) if split else 0.0)
    codes, scales = backend.quantize_rows_e4m3(hi, lo)
    ref_codes, ref_scales = backend.quantize_fp8(xf)
    assert np.array_equal(scales.view(np.uint32), ref_scales.view(np.uint32))
    mism = np.count_nonzero(codes != ref_codes)
    print(f"quantise {rows}x{cols} split={split}: {mism} code mismatches")
    assert mism == 0
    # Round trip within half an e4m3 step of each value.
    back = _decode_e4m3(codes) * scales[:, None]
    assert np.all(np.abs(back - xf) <= np.abs(xf) / 16 + scales[:, None] * 2.0 ** -10)


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 256), (2048, 1024, 1024), (2304, 1536, 1536)])
@pytest.mark.parametrize("act", ["none", "mish"])
def test_fp8_gemm_against_fp64(m, n, k, act):
    """4096 x 4096 fills whole rounds of 256 x 256 tiles; the others take the
    128 x 128 fp8 tiles."""
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    ac, asc = backend.quantize_fp8(a)
    wc, wsc = backend.quantize_fp8(w)
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    got = backend.gemm_fp8(ac, asc, wc, wsc, bias, act=act)
    x = (_decode_e4m3(ac) * asc[:, None].astype(np.float64)) @ \
        (_decode_e4m3(wc) * wsc[:, None].astype(np.float64)).T + bias
    ref = x * np.tanh(np.log1p(np.exp(x))) if act == "mish" else x
    err = np.abs(got - ref).max()
    print(f"fp8 gemm {m}x{n}x{k} {act}: max-abs {err:.2e} (|ref| max {np.abs(ref).max():.2f})")
    # The fp8 MFMA's sums of products land within 2-3e-5 of their fp64
    # values here, three orders of magnitude below an e4m3 step (2^-4).
    assert err <= 1e-4 * max(1.0, np.abs(ref).max())


def test_fp8_gemm_rejects_small_m():
    codes = np.zeros((64, 128), np.uint8)
    with pytest.raises(RuntimeError):
        backend.gemm_fp8(codes, np.ones(64, np.float32), codes, np.ones(64, np.float32))
