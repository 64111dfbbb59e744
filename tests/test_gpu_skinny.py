"""The few-row GEMM (skinny_gemm.hip; the batch-1 smolgen chain) against
fp64 references of the same bf16 operands, through mfh_debug_skinny_gemm.

Covers both activation operands (bf16 planes, and the LayerNorm of fp32
rows applied as the rows are loaded, reference cpu_network.cpp:424-460),
split and single precision, the three outputs (bf16 planes, fp32, residual),
the per-workgroup row statistics, the stored normalised rows, one and two
16-column tiles per workgroup, 1 / 20 / 32 / 64 rows, and the smolgen
global projection's row segments (each A row one head's slice of a longer
source row, normalised over the whole source row)."""

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
    return (np.asarray(b).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _split(x):
    hi = _bits(x)
    lo = _bits(np.asarray(x, np.float32) - _f(hi).astype(np.float32))
    return hi, lo


def _mish(x):
    return x * np.tanh(np.log1p(np.exp(x)))


def _layernorm(x, gamma, beta, eps):
    x = x.astype(np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = (x * x).mean(axis=-1, keepdims=True) - mean * mean
    return (x - mean) / np.sqrt(np.maximum(var, 0.0) + eps) * gamma + beta


@pytest.mark.parametrize("m,n,k,split", [(1, 256, 2048, True), (20, 96, 1024, False),
                                         (64, 3104, 1024, True), (64, 8192, 256, True),
                                         (32, 64, 256, False)])
def test_planes_bf16_output(m, n, k, split):
    rng = np.random.default_rng(m * 7 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    hi, lo = _split(a)
    w = _bits(rng.standard_normal((n, k)) / np.sqrt(k))
    bias = rng.standard_normal(n).astype(np.float32)
    out_hi, out_lo = backend.skinny_gemm(w, a_bits=hi, a_lo_bits=lo if split else None,
                                         bias=bias, act="mish", out_mode="bf16", want_lo=True)
    aa = _f(hi) + (_f(lo) if split else 0.0)
    ref = _mish(aa @ _f(w).T + bias)
    got = _f(out_hi) + _f(out_lo)
    err = np.abs(got - ref).max()
    print(f"planes m={m} n={n} k={k} split={split}: max-abs {err:.2e}")
    assert err <= 2e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("m,n,k", [(64, 1024, 1024), (64, 1024, 1536), (1, 8192, 256)])
@pytest.mark.parametrize("resid_kind", ["planes", "f32"])
def test_residual_output_and_row_statistics(m, n, k, resid_kind):
    rng = np.random.default_rng(n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    hi, lo = _split(a)
    w = _bits(rng.standard_normal((n, k)) / np.sqrt(k))
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    r = rng.standard_normal((m, n)).astype(np.float32)
    if resid_kind == "planes":
        rh, rl = _split(r)
        resid, rr = (rh, rl), _f(rh) + _f(rl)
    else:
        resid, rr = r, r.astype(np.float64)
    out, stats = backend.skinny_gemm(w, a_bits=hi, a_lo_bits=lo, bias=bias, out_mode="resid",
                                     resid=resid, alpha=0.7)
    ref = rr + 0.7 * ((_f(hi) + _f(lo)) @ _f(w).T + bias)
    err = np.abs(out - ref).max()
    # Row statistics: the parts together cover every column once.
    s = stats[:, :, 0].astype(np.float64).sum(axis=0)
    ss = stats[:, :, 1].astype(np.float64).sum(axis=0)
    serr = np.abs(s - out.astype(np.float64).sum(axis=1)).max()
    sserr = np.abs(ss - (out.astype(np.float64) ** 2).sum(axis=1)).max()
    print(f"resid {resid_kind} m={m} n={n} k={k}: {err:.2e}, "
          f"stats {serr:.2e} / {sserr:.2e}, "
          f"{stats.shape[0]} parts")
    assert err <= 2e-5 * max(1.0, np.abs(ref).max())
    assert serr <= 1e-4 * n and sserr <= 1e-4 * n * max(1.0, np.abs(out).max()) ** 2


@pytest.mark.parametrize("m,n,k,split", [(64, 3104, 1024, True), (64, 1536, 1024, False),
                                         (1, 8192, 256, True), (1, 8192, 256, False)])
def test_layernorm_operand(m, n, k, split):
    """A = LayerNorm(x) on the fly; the normalised rows are stored too."""
    rng = np.random.default_rng(k + m)
    x = (rng.standard_normal((m, k)) * 2.0 + 0.5).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(k)).astype(np.float32)
    w = _bits(rng.standard_normal((n, k)) / np.sqrt(k))
    bias = rng.standard_normal(n).astype(np.float32)
    ln = dict(x=x, gamma=gamma, beta=beta, eps=1e-3, rows=m, split=split)
    out_hi, out_lo, (y_hi, y_lo, y32) = backend.skinny_gemm(
        w, ln=ln, bias=bias, out_mode="bf16", want_lo=True)
    y_ref = _layernorm(x, gamma, beta, 1e-3)
    yerr = np.abs(y32 - y_ref).max()
    ysplit = np.abs(_f(y_hi) + _f(y_lo) - y32).max()
    # The product of the operand the kernel used (its own stored rows).
    aa = _f(y_hi) + (_f(y_lo) if split else 0.0)
    ref = aa @ _f(w).T + bias
    err = np.abs(_f(out_hi) + _f(out_lo) - ref).max()
    print(f"ln m={m} n={n} k={k} split={split}: y {yerr:.2e} (hi+lo {ysplit:.2e}), out {err:.2e}")
    # hi + lo holds a value to about 2^-17 of its size.
    assert yerr <= 1e-4 and ysplit <= 2e-5 * max(1.0, np.abs(y32).max())
    assert err <= 2e-5 * max(1.0, np.abs(ref).max())
    # Against the fp64 chain end to end.
    full = (y_ref if split else _f(_bits(y_ref))) @ _f(w).T + bias
    assert np.abs(_f(out_hi) + _f(out_lo) - full).max() <= 2e-3 * max(1.0, np.abs(full).max())


@pytest.mark.parametrize("heads,gen,n,split", [(32, 256, 4096, True), (32, 256, 4096, False),
                                               (8, 64, 4096, True)])
def test_layernorm_row_segments(heads, gen, n, split):
    """The smolgen global projection at one position: A row h is head h's
    gen-wide slice of the dense2 row, normalised over the whole row."""
    rng = np.random.default_rng(heads + gen)
    x = rng.standard_normal((1, heads * gen)).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(heads * gen)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(heads * gen)).astype(np.float32)
    w = _bits(rng.standard_normal((n, gen)) / np.sqrt(gen))
    ln = dict(x=x, gamma=gamma, beta=beta, eps=1e-3, rows=heads, rows_per_src=heads,
              split=split)
    out, stats = backend.skinny_gemm(w, ln=ln, out_mode="f32")
    y = _layernorm(x, gamma, beta, 1e-3).reshape(heads, gen)
    a = y if split else _f(_bits(y))
    ref = a @ _f(w).T
    err = np.abs(out - ref).max()
    print(f"segments heads={heads} gen={gen} split={split}: {err:.2e}")
    assert err <= 2e-3 * max(1.0, np.abs(ref).max())


def test_rejects_bad_shapes():
    w = _bits(np.ones((64, 64), np.float32))
    a = _bits(np.ones((65, 64), np.float32))
    with pytest.raises(RuntimeError):
        backend.skinny_gemm(w, a_bits=a)  # more than 64 rows
