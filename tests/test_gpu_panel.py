"""Row-panel GEMM (PanelGemmKernel) through the C ABI against float64
numpy: the fused residual + LayerNorm epilogue (reference
cpu_network.cpp:1256-1259 / 1318-1397 then 1399-1457: LN(x + alpha * y),
mean = sum/N, var = sum(x^2)/N - mean^2 clamped at 0, eps inside the square
root) and the bias + activation epilogue, for every panel width, split and
single activations, bf16 and e4m3 weights, and row counts that are not a
multiple of the 64-row panel."""

import numpy as np
import pytest

from metalfish_amd import backend, synth

pytestmark = pytest.mark.gpu


def _bf16_bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _split(x):
    hi = _bf16_bits(x)
    lo = _bf16_bits(x.astype(np.float32) - _f32(hi))
    return hi, lo


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if backend.device_count() < 1:
        pytest.fail("GPU tests need an MI355X; none visible")


def _operands(rng, m, n, k, split, w8):
    x = rng.standard_normal((m, k)).astype(np.float32)
    if split:
        a, a_lo = _split(x)
        a_val = _f32(a).astype(np.float64) + _f32(a_lo)
    else:
        a, a_lo = _bf16_bits(x), None
        a_val = _f32(a).astype(np.float64)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    if w8:
        codes, scale = backend.quantize_fp8(w)
        w_val = synth.e4m3_values()[codes].astype(np.float64) * scale[:, None]
        wargs = dict(w8_codes=codes, wscale=scale)
    else:
        wb = _bf16_bits(w)
        w_val = _f32(wb).astype(np.float64)
        wargs = dict(w_bits=wb)
    bias = rng.standard_normal(n).astype(np.float32)
    return a, a_lo, a_val, wargs, w_val, bias


@pytest.mark.parametrize("m,n,k,split,w8,resid", [
    (100, 256, 256, False, False, "f32"),     # panel width 2, ragged last panel
    (130, 512, 512, True, False, "pair"),     # width 4
    (64, 768, 1536, True, True, "f32"),       # width 6, e4m3 weights
    (200, 1024, 1024, True, False, "pair"),   # width 8, the BT4 out-projection
    (4096, 1024, 1536, True, False, "pair"),  # the BT4 FFN2 at 64 positions
    (1000, 1024, 1536, False, True, "f32"),   # single activations, e4m3
])
def test_panel_layernorm_against_fp64(m, n, k, split, w8, resid):
    rng = np.random.default_rng(m + n + k)
    a, a_lo, a_val, wargs, w_val, bias = _operands(rng, m, n, k, split, w8)
    r = rng.standard_normal((m, n)).astype(np.float32)
    if resid == "pair":
        r_hi, r_lo = _split(r)
        r_val = _f32(r_hi).astype(np.float64) + _f32(r_lo)
        rargs = dict(resid_hi=r_hi, resid_lo=r_lo)
    else:
        r_val = r.astype(np.float64)
        rargs = dict(resid32=r)
    gamma = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(n)).astype(np.float32)
    alpha, eps = 0.7, 1e-3
    hi, lo, y32 = backend.panel_gemm(a, a_lo_bits=a_lo, bias=bias, **wargs,
                                     layernorm=dict(gamma=gamma, beta=beta, eps=eps,
                                                    alpha=alpha, **rargs))
    x = r_val + alpha * (a_val @ w_val.T + bias)
    mean = x.mean(axis=1, keepdims=True)
    var = np.maximum((x * x).mean(axis=1, keepdims=True) - mean * mean, 0)
    ref = (x - mean) / np.sqrt(var + eps) * gamma + beta
    err = np.abs(y32 - ref).max()
    print(f"panel LN m={m} n={n} k={k} split={split} w8={w8}: max-abs {err:.2e}")
    # fp32 accumulation over k terms of size ~1: |x| error ~1e-5, divided by
    # the row's standard deviation (~1.2 here).
    assert err <= 2e-4
    # The bf16 planes are the rounding of the fp32 output and its remainder.
    assert np.array_equal(hi, _bf16_bits(y32))
    assert np.array_equal(lo, _bf16_bits(y32 - _f32(hi)))


@pytest.mark.parametrize("m,n,k,split,w8,act", [
    (100, 1536, 256, True, False, "mish"),    # two panels of 768
    (70, 3072, 128, False, False, "none"),    # three panels of 1024
    (300, 2048, 1024, True, True, "swish"),   # two panels of 1024, e4m3, runtime act
])
def test_panel_bias_activation_against_fp64(m, n, k, split, w8, act):
    rng = np.random.default_rng(m * 3 + n + k)
    a, a_lo, a_val, wargs, w_val, bias = _operands(rng, m, n, k, split, w8)
    hi, lo = backend.panel_gemm(a, a_lo_bits=a_lo, bias=bias, act=act, **wargs)
    y = a_val @ w_val.T + bias
    if act == "mish":
        y = y * np.tanh(np.log1p(np.exp(y)))
    elif act == "swish":
        y = y / (1 + np.exp(-y))
    got = _f32(hi).astype(np.float64) + _f32(lo)
    err = np.abs(got - y).max()
    print(f"panel act m={m} n={n} k={k} split={split} w8={w8} {act}: max-abs {err:.2e}")
    assert err <= 1e-4 * max(1.0, np.abs(y).max())


def _rounding_cases(rng, n):
    """float32 values whose bf16 rounding the split must get right: random
    magnitudes over the whole range, exact ties (low half 0x8000, even and
    odd kept bits), denormals and denormal ties, both signs, zeros."""
    sign = rng.integers(0, 2, n, dtype=np.uint32) << 31
    hi16 = rng.integers(0, 0x7F7F, n, dtype=np.uint32)
    kinds = [
        (hi16 << 16) | rng.integers(0, 1 << 16, n, dtype=np.uint32),   # anything finite
        (hi16 << 16) | 0x8000,                                           # ties
        rng.integers(1, 1 << 23, n, dtype=np.uint32),                    # denormals
        (rng.integers(0, 0x80, n, dtype=np.uint32) << 16) | 0x8000,      # denormal ties
    ]
    bits = np.concatenate([k | sign for k in kinds])
    bits[:4] = [0, 0x80000000, 0x00008000, 0x7F7F7FFF]
    return bits.view(np.float32)


def test_bf16_split_rounding_bit_exact():
    """The epilogues' bf16 hi + lo split (hi = bf16(v), lo = bf16(v - hi),
    round to nearest even on gfx950's v_cvt_pk_bf16_f32) against the integer
    rounding on the host, bit for bit: a zero product plus a bias of crafted
    values, through the row-panel GEMM's bias epilogue (the helper the tiled
    GEMM, attention and the panel share)."""
    rng = np.random.default_rng(11)
    vals = _rounding_cases(rng, 3072)
    a = np.zeros((64, 128), np.uint16)
    w = np.zeros((3072, 128), np.uint16)
    for c in range(0, vals.size, 3072):
        bias = vals[c:c + 3072]
        hi, lo = backend.panel_gemm(a, w_bits=w, bias=bias)
        y = np.float32(0) + bias
        want_hi, want_lo = _split(y)
        bad = np.flatnonzero((hi != want_hi[None, :]).any(0) | (lo != want_lo[None, :]).any(0))
        assert bad.size == 0, [(hex(int(y.view(np.uint32)[i])), hex(int(hi[0, i])),
                                hex(int(want_hi[i])), hex(int(lo[0, i])), hex(int(want_lo[i])))
                               for i in bad[:8]]


def test_panel_rejects_bad_shapes():
    a = np.zeros((64, 256), np.uint16)
    w = np.zeros((320, 256), np.uint16)  # 320 columns: no panel width
    with pytest.raises(RuntimeError, match="panel"):
        backend.panel_gemm(a, w_bits=w)
    w = np.zeros((512, 256), np.uint16)
    with pytest.raises(RuntimeError, match="LayerNorm"):
        backend.panel_gemm(a, w_bits=w, layernorm=dict(gamma=np.ones(512), beta=np.zeros(512)))
