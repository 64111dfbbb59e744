"""FP8 (OCP e4m3) weight storage: the host quantiser of the C ABI and the
numpy one the tests use for the oracle's weights, both against a
brute-force nearest-value encoder written from the format definition
(bias 7, 3 mantissa bits, subnormals m * 2^-9, largest finite 448, ties to
the even code)."""

import numpy as np
import pytest

from metalfish_amd import backend, synth


@pytest.fixture(autouse=True)
def _experimental_fp8(monkeypatch):
    """The FP8 precision is below the parity gates, so mfh_net_create takes
    it only on explicit request; these tests make that request."""
    monkeypatch.setenv("METALFISH_HIP_EXPERIMENTAL_FP8", "1")


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


def _fp8_parity(spec_name, n, seed=0, batch=None, precision="bf16x2"):
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
    net = backend.create_network(spec, weights, max_batch=batch, device=0, weights_dtype="fp8",
                                 precision=precision)
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
    print(f"fp8 {precision} {spec_name} x{n}: policy max-abs {perr:.3e} wdl max-abs {werr:.3e} top1 {agree:.3f}")
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


@pytest.mark.gpu
@pytest.mark.parametrize("n,batch", [(40, None), (40, 128)])
def test_fp8_activation_parity(n, batch):
    """The FP8 precision (e4m3 activations into the body's Q|K|V, out-
    projection and FFN GEMMs from 2048 token rows) against the oracle on the
    same dequantised weights.

    It does not meet the parity gates (top-1 >= 99.5 %, policy max-abs
    <= 2e-2, WDL <= 5e-3): on the random-init BT4 net it measured top-1
    0.825 / 0.789, policy max-abs 0.15 / 0.18 and WDL max-abs 1.6e-2 /
    1.1e-2 at 40 positions / a batch of 128, while each fp8 GEMM matches
    fp64 of its codes (test_fp8_precision_layer_integration): the loss is
    the 3-bit mantissa of the activations compounding over 15 layers.  The
    bounds below only catch wiring regressions (which give top-1 near chance,
    a few percent): any change of fp32 summation order anywhere in the net
    moves some activations across an e4m3 rounding boundary, and top-1 on 40
    positions has measured anywhere from 0.65 to 0.83 across such changes."""
    if backend.device_count() < 1:
        pytest.fail("GPU tests need an MI355X; none visible")
    perr, werr, agree = _fp8_parity("bt4", n, batch=batch, precision="fp8")
    assert perr <= 0.3 and werr <= 0.04 and agree >= 0.5


@pytest.mark.gpu
def test_fp8_precision_below_2048_rows_is_bf16():
    """Below 2048 token rows the FP8 precision runs the BF16 path: the same
    bits as a BF16-precision net on the same e4m3 weights.  Against the
    oracle it is held to the single-bf16 bounds (policy max-abs 3e-2, WDL
    5e-3; top-1 reported, since the random-init net has near-tied legal
    logits that single-bf16 rounding reorders)."""
    import oracle

    if backend.device_count() < 1:
        pytest.fail("GPU tests need an MI355X; none visible")
    spec = synth.SPECS["bt4"]
    weights = synth.make_weights(spec, seed=0, fp8=True)
    planes, legal = synth.playout_positions(8, seed=0)
    out = {}
    for precision in ("fp8", "bf16"):
        net = backend.create_network(spec, weights, max_batch=8, device=0, weights_dtype="fp8",
                                     precision=precision)
        out[precision] = net.evaluate_batch(planes)
        net.close()
    for k in ("policy", "wdl"):
        assert np.array_equal(out["fp8"][k].view(np.uint32), out["bf16"][k].view(np.uint32)), k
    ref = oracle.OracleNet(oracle.NetFormat(body_heads=spec.heads), weights).evaluate_batch(planes)
    perr = np.abs(out["fp8"]["policy"] - ref["policy"]).max()
    werr = np.abs(out["fp8"]["wdl"] - ref["wdl"]).max()
    agree = np.mean([np.argmax(out["fp8"]["policy"][i, l[l >= 0]]) ==
                     np.argmax(ref["policy"][i, l[l >= 0]]) for i, l in enumerate(legal)])
    print(f"fp8 below 2048 rows: policy max-abs {perr:.3e} wdl max-abs {werr:.3e} top1 {agree:.3f}")
    assert perr <= 3e-2 and werr <= 5e-3


def test_fp8_precision_needs_fp8_weights():
    spec = synth.SPECS["cpu_plumbing"]
    weights = synth.make_weights(spec, seed=0)
    with pytest.raises(RuntimeError, match="FP8 precision needs FP8"):
        backend.create_network(spec, weights, max_batch=4, device=-1, precision="fp8")


def test_fp8_precision_needs_explicit_request(monkeypatch):
    """Without METALFISH_HIP_EXPERIMENTAL_FP8=1 the FP8 precision is refused
    at creation with a message that says why; e4m3 weights with the bf16x2
    precision need no request."""
    monkeypatch.delenv("METALFISH_HIP_EXPERIMENTAL_FP8")
    spec = synth.SPECS["cpu_plumbing"]
    weights = synth.make_weights(spec, seed=0, fp8=True)
    with pytest.raises(RuntimeError, match="experimental and below the parity gates"):
        backend.create_network(spec, weights, max_batch=4, device=-1, precision="fp8",
                               weights_dtype="fp8")


def _e4m3_decode(codes):
    v = synth.e4m3_values().astype(np.float64)
    return v[np.asarray(codes)]


def _bits_f64(b):
    return (np.asarray(b).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _to_bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _ln(x, g, b, eps):
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * g + b


@pytest.mark.gpu
def test_fp8_precision_layer_integration():
    """One BT4 encoder layer in the FP8 precision at 32 positions (2048 token
    rows), step by step against fp64 on the host: each e4m3 GEMM input is
    the row quantisation of the tensor it stands for (bit for bit), and each
    GEMM output is the product of those codes with the layer's weights
    (Q|K|V, out-projection through the first LayerNorm, FFN1 with Mish,
    FFN2's residual sum, the second LayerNorm)."""
    if backend.device_count() < 1:
        pytest.fail("GPU tests need an MI355X; none visible")
    spec = synth.SPECS["bt4"]
    w = synth.make_weights(spec, seed=5, fp8=True)
    b, e, f = 32, spec.embedding, spec.ffn
    m = b * 64
    net = backend.create_network(spec, w, max_batch=b, device=0, weights_dtype="fp8",
                                 precision="fp8")
    rng = np.random.default_rng(11)
    x_bits = _to_bits(rng.standard_normal((m, e)))
    net.encoder_layer_ms(b, 0, 1, x_bits)
    get = net.debug_tensor
    qkv = _bits_f64(get("qkv", (m, 3 * e), np.uint16))
    ctx_bits = get("ctx", (m, e), np.uint16)
    hid_bits = get("hid", (m, f), np.uint16)
    pre = get("pre", (m, e), np.float32).astype(np.float64)
    body = get("body", (m, e), np.float32).astype(np.float64)
    act8, act_s = get("act_e4m3", (m, e), np.uint8), get("act_scale", (m,), np.float32)
    ctx8, ctx_s = get("ctx_e4m3", (m, e), np.uint8), get("ctx_scale", (m,), np.float32)
    hid8, hid_s = get("hid_e4m3", (m, f), np.uint8), get("hid_scale", (m,), np.float32)
    net.close()

    p = "body.encoder.0."
    W = lambda n: w[p + n].astype(np.float64)
    alpha = float(np.float32(2.0 * spec.layers) ** np.float32(-0.25))
    eps = 1e-6 if spec.pe_map else 1e-3
    x = _bits_f64(x_bits)

    def deq(codes, s):
        return _e4m3_decode(codes) * s.astype(np.float64)[:, None]

    def near_bf16(got, ref):
        # bf16 rounding of the output (2^-9 relative) plus the fp8 MFMA's
        # summation error (1e-4 of the largest output).
        return np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-4 * np.abs(ref).max())

    # Q|K|V from the quantised layer input.
    xq, xs = backend.quantize_fp8(x.astype(np.float32))
    wqkv = np.concatenate([W("mha.q_w"), W("mha.k_w"), W("mha.v_w")])
    bqkv = np.concatenate([W("mha.q_b"), W("mha.k_b"), W("mha.v_b")])
    ref_qkv = deq(xq, xs) @ wqkv.T + bqkv
    assert near_bf16(qkv, ref_qkv), np.abs(qkv - ref_qkv).max()
    # Out-projection input: the attention output, quantised bit for bit.
    cq, cs = backend.quantize_fp8(_bits_f64(ctx_bits).astype(np.float32))
    assert np.array_equal(ctx8, cq) and np.array_equal(ctx_s.view(np.uint32), cs.view(np.uint32))
    resid1 = _ln(x + alpha * (deq(ctx8, ctx_s) @ W("mha.dense_w").T + W("mha.dense_b")),
                 W("ln1_gammas"), W("ln1_betas"), eps)
    # FFN1 input: the first LayerNorm's bf16 rows, quantised (a host row
    # that rounds to other bf16 values than the device's fp32 LayerNorm can
    # differ in a few codes).
    aq, _ = backend.quantize_fp8(_bits_f64(_to_bits(resid1)).astype(np.float32))
    agree = np.mean(act8 == aq)
    print(f"FFN1 input codes equal to the host's: {agree:.6f}")
    assert agree >= 0.999
    lin1 = deq(act8, act_s) @ W("ffn.dense1_w").T + W("ffn.dense1_b")
    ref_hid = lin1 * np.tanh(np.log1p(np.exp(lin1)))
    assert near_bf16(_bits_f64(hid_bits), ref_hid), np.abs(_bits_f64(hid_bits) - ref_hid).max()
    hq, hs = backend.quantize_fp8(_bits_f64(hid_bits).astype(np.float32))
    assert np.array_equal(hid8, hq) and np.array_equal(hid_s.view(np.uint32), hs.view(np.uint32))
    ref_pre = resid1 + alpha * (deq(hid8, hid_s) @ W("ffn.dense2_w").T + W("ffn.dense2_b"))
    perr = np.abs(pre - ref_pre).max()
    berr = np.abs(body - _ln(pre, W("ln2_gammas"), W("ln2_betas"), eps)).max()
    print(f"FFN2 residual sum max-abs {perr:.2e}, LayerNorm {berr:.2e}")
    assert perr <= 1e-4 * np.abs(ref_pre).max() and berr <= 1e-4


def test_fp8_precision_rejects_widths_the_quantiser_cannot_take():
    """FFN 2560 (> 2048 values per row) is refused at creation, before any
    device work."""
    spec = synth.NetSpec(**{**synth.SPECS["cpu_plumbing"].__dict__, "ffn": 2560})
    weights = synth.make_weights(spec, seed=0, fp8=True)
    with pytest.raises(RuntimeError, match="multiples of 128 up to 2048"):
        backend.create_network(spec, weights, max_batch=4, device=-1, precision="fp8",
                               weights_dtype="fp8")
