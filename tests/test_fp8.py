"""FP8 (OCP e4m3) weight storage: the host quantiser of the C ABI and the
numpy one the tests use for the oracle's weights, both against a
brute-force nearest-value encoder written from the format definition
(bias 7, 3 mantissa bits, subnormals m * 2^-9, largest finite 448, ties to
the even code)."""

import numpy as np
import pytest

from metalfish_amd import backend, synth


def _finite_table():
    vals = []
    for c in range(0x7F):  # positive codes, 0x7F is NaN
        e, m = c >> 3, c & 7
        vals.append((1 + m / 8.0) * 2.0 ** (e - 7) if e else m * 2.0 ** -9)
    return np.array(vals)


def _brute_encode(x):
    table = _finite_table()
    out = np.empty(x.shape, np.uint8)
    for i, v in np.ndenumerate(x.astype(np.float64)):
        a = min(abs(v), 448.0)
        d = np.abs(table - a)
        best = np.flatnonzero(d == d.min())
        code = best[0] if len(best) == 1 else best[(best & 1) == 0][0]
        out[i] = code | (0x80 if np.signbit(v) else 0)
    return out


def test_value_table():
    v = synth.e4m3_values()
    assert v[0x7E] == 448 and v[0x01] == 2.0 ** -9 and v[0x08] == 2.0 ** -6
    assert v[0x38] == 1.0 and v[0xFE] == -448 and np.isnan(v[0x7F]) and np.isnan(v[0xFF])


def test_encoders_match_brute_force():
    rng = np.random.default_rng(7)
    table = _finite_table()
    mids = (table[1:] + table[:-1]) / 2  # exact ties
    x = np.concatenate([
        rng.standard_normal(4000) * 50, rng.standard_normal(2000) * 0.01,
        table, -table, mids, -mids, [0.0, -0.0, 448.0, 460.0, 463.9, 464.0, 1e4, -1e4,
                                     2.0 ** -10, 3 * 2.0 ** -11, 1e-30]]).astype(np.float32)
    ref = _brute_encode(x)
    assert np.array_equal(synth.e4m3_encode(x), ref)


def test_row_quantisation_library_matches_numpy():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((37, 200)) / 14).astype(np.float32)
    w[5] = 0.0
    w[6, :3] = [1e-7, -2e-8, 3.0]
    codes, scale = backend.quantize_fp8(w)
    c2, s2, deq = synth.quantize_fp8_rows(w)
    assert np.array_equal(codes, c2)
    assert np.array_equal(scale.view(np.uint32), s2.view(np.uint32))
    assert scale[5] == 1.0 and not codes[5].any()
    # Re-quantising the dequantised values gives the same codes: the weights
    # handed to an fp8 net are exactly what it stores.
    c3, _, deq3 = synth.quantize_fp8_rows(deq)
    assert np.array_equal(c3, codes)
    assert np.allclose(deq3, deq, rtol=2 ** -22, atol=0)


def _fp8_parity(spec_name, n, seed=0, batch=None):
    """Parity of an fp8 net on n positions against the oracle; with `batch`,
    the positions fill a batch of that size cyclically (large batches take
    the row-panel GEMMs) and every copy is compared."""
    import oracle

    spec = synth.SPECS[spec_name]
    weights = synth.make_weights(spec, seed=seed, fp8=True)
    planes, legal = synth.playout_positions(n, seed=seed)
    ref = oracle.OracleNet(oracle.NetFormat(body_heads=spec.heads), weights).evaluate_batch(planes)
    batch = batch or n
    idx = np.arange(batch) % n
    net = backend.create_network(spec, weights, max_batch=batch, device=0, weights_dtype="fp8")
    gpu = net.evaluate_batch(planes[idx])
    net.close()
    planes, legal = planes[idx], legal[idx]
    ref = {k: v[idx] for k, v in ref.items()}
    n = batch
    perr = np.abs(gpu["policy"] - ref["policy"]).max()
    werr = np.abs(gpu["wdl"] - ref["wdl"]).max()
    agree = np.mean([legal[i][legal[i] >= 0][np.argmax(gpu["policy"][i, legal[i][legal[i] >= 0]])] ==
                     legal[i][legal[i] >= 0][np.argmax(ref["policy"][i, legal[i][legal[i] >= 0]])]
                     for i in range(n)])
    print(f"fp8 {spec_name} x{n}: policy max-abs {perr:.3e} wdl max-abs {werr:.3e} top1 {agree:.3f}")
    return perr, werr, agree


@pytest.mark.gpu
@pytest.mark.parametrize("spec_name,n,batch", [("cpu_plumbing", 16, None), ("bt4", 8, None),
                                              ("bt4", 40, None), ("bt4", 40, 128)])
def test_fp8_weight_parity(spec_name, n, batch):
    """fp8-weight nets (bf16x2 activations) against the oracle running on the
    same dequantised weights; 40 BT4 positions reach the large-M tiles, a
    batch of 128 the row-panel GEMMs with the fused LayerNorm."""
    if backend.device_count() < 1:
        pytest.fail("GPU tests need an MI355X; none visible")
    perr, werr, agree = _fp8_parity(spec_name, n, batch=batch)
    assert perr <= 1e-3 and werr <= 1e-4 and agree == 1.0
