"""The BF16X2_FP8LO precision: activations hi (bf16) + lo (OCP e4m3 codes of
lo * 2^10) into the encoder GEMMs, each GEMM the hi product on the bf16 MFMA
plus the lo product on the fp8 MFMA (v_mfma_f32_16x16x128_f8f6f4).

* The GEMM kernel (mfh_debug_gemm_lo8) against float64 on random operands:
  acc = A.W^T + dec(A_lo8).dec(W_lo8)^T, out = act(acc * wscale + bias), at
  the encoder shapes of batches 128 and 256 and at a ragged shape (partial
  tiles on both sides); its bf16 + e4m3-lo output form decodes back to the
  fp32 result.
* The forward: below 8192 token rows the precision is BF16X2 bit for bit
  (the scaled weights and column scales are exact powers of two); from 8192
  rows it meets the parity gates against the CPU oracle (policy max-abs
  <= 2e-2, WDL <= 5e-3, same top-1 legal move on >= 99.5 % of positions)
  on bf16 and on e4m3 weights, and graph replays equal the eager forward.
"""

import numpy as np
import pytest

import gpu_util
from metalfish_amd import backend, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if backend.device_count() < 1:
        pytest.fail("GPU tests need an MI355X; none visible")


E4M3 = synth.e4m3_values().astype(np.float64)


def _bf16_bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _f64(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _codes(rng, shape):
    """Random finite e4m3 codes (0x7F / 0xFF are NaN)."""
    c = rng.integers(0, 256, size=shape, dtype=np.uint8)
    return np.where((c & 0x7F) == 0x7F, c ^ 0x01, c).astype(np.uint8)


@pytest.mark.parametrize("m,n,k", [
    (16384, 3072, 1024),  # Q|K|V, batch 256
    (16384, 1024, 1536),  # FFN2
    (8192, 1536, 1024),   # FFN1, batch 128
    (1000, 200, 384),     # ragged: partial tiles in M and N
])
def test_gemm_lo8_against_fp64(m, n, k):
    rng = np.random.default_rng(m + 7 * n + k)
    a = _bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    w = _bf16_bits(rng.standard_normal((n, k), dtype=np.float32) * 300)
    a8, w8 = _codes(rng, (m, k)), _codes(rng, (n, k))
    ws = (2.0 ** rng.integers(-20, -8, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    got = backend.gemm_lo8(a, a8, w, w8, ws, bias)
    rows = np.unique(np.concatenate([rng.integers(0, m, 256), [0, m - 1]]))
    acc = _f64(a[rows]) @ _f64(w).T + E4M3[a8[rows]] @ E4M3[w8].T
    terms = np.abs(_f64(a[rows])) @ np.abs(_f64(w)).T + np.abs(E4M3[a8[rows]]) @ np.abs(E4M3[w8]).T
    ref = acc * ws + bias
    err = np.abs(got[rows] - ref)
    # fp32 accumulation: ~2^-24 per addition of the magnitudes summed.
    bound = 4 * k * 2.0 ** -24 * terms * ws + 1e-6
    print(f"lo8 gemm {m}x{n}x{k}: max-abs {err.max():.3e}, worst err / bound "
          f"{(err / bound).max():.3f}", flush=True)
    assert (err <= bound).all()


def test_gemm_lo8_bf16_output_codes():
    """bf16 output with e4m3 lo codes (the FFN1 epilogue of the precision):
    hi is the bf16 rounding of the fp32 result (Mish applied) and the codes
    decode to (result - hi) * 2^10 within e4m3 rounding."""
    m, n, k = 8192, 1536, 1024
    rng = np.random.default_rng(5)
    a = _bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    w = _bf16_bits(rng.standard_normal((n, k), dtype=np.float32) / 32)
    a8, w8 = _codes(rng, (m, k)) & 0xBF, _codes(rng, (n, k)) & 0xBF  # smaller codes
    ws = np.full(n, 1.0, np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    f32 = backend.gemm_lo8(a, a8, w, w8, ws, bias, act="mish")
    hi, lo8 = backend.gemm_lo8(a, a8, w, w8, ws, bias, act="mish", bf16_out=True)
    assert np.array_equal(hi, _bf16_bits(f32))
    lo = f32.astype(np.float64) - _f64(hi)
    dec = E4M3[lo8] / 1024.0
    # Half an e4m3 ulp (2^-4 relative) or half the smallest subnormal step.
    assert (np.abs(dec - lo) <= np.abs(lo) * 2.0 ** -4 + 2.0 ** -20).all()


# ---- The forward ----------------------------------------------------------

POLICY_TOL = 2e-2
WDL_TOL = 5e-3
TOP1_GATE = 0.995


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _top1(pol, ref_pol, legal):
    agree = 0
    for i in range(pol.shape[0]):
        idx = legal[i][legal[i] >= 0]
        agree += int(idx[np.argmax(pol[i, idx])] == idx[np.argmax(ref_pol[i, idx])])
    return agree / pol.shape[0]


@pytest.fixture(scope="module")
def positions():
    planes, legal = synth.playout_positions(256, seed=0)
    masks, values = backend.pack_planes(planes)
    return dict(planes=planes, legal=legal, masks=masks, values=values)


def _device_runs(net, masks, values, runs=4):
    """mfh_net_eval_device on a caller stream: eager run, graph capture and
    replays; returns the outputs of each call."""
    B = masks.shape[0]
    dev = gpu_util.DeviceBuffers()
    stream = dev.stream()
    pol0 = np.zeros((B, 1858), np.float32)
    wdl0 = np.zeros((B, 3), np.float32)
    d_m, d_v = dev.put(masks), dev.put(values)
    d_p, d_w = dev.put(pol0), dev.put(wdl0)
    out = []
    for _ in range(runs):
        net.eval_device(B, d_m, d_v, d_p, d_w, stream=stream)
        dev.sync(stream)
        out.append((dev.get(d_p, pol0), dev.get(d_w, wdl0)))
    dev.free()
    return out


def test_below_threshold_equals_bf16x2(positions):
    """At 64 positions (4096 rows) the precision runs the BF16X2 forward on
    power-of-two-scaled weights: the same bits as a BF16X2 net."""
    spec = synth.SPECS["bt4"]
    weights = synth.make_weights(spec, seed=0)
    s = slice(0, 64)
    out = {}
    for precision in ("bf16x2", "bf16x2_fp8lo"):
        net = backend.create_network(spec, weights, max_batch=64, device=0, precision=precision)
        out[precision] = net.eval_packed(positions["masks"][s], positions["values"][s])
        net.close()
    for k in range(2):
        assert np.array_equal(_bits(out["bf16x2"][k]), _bits(out["bf16x2_fp8lo"][k]))


@pytest.mark.timeout(900)
@pytest.mark.parametrize("weights_dtype,batch", [("bf16", 256), ("bf16", 128), ("fp8", 1024)])
def test_forward_gates(positions, bt4_bench_oracle, weights_dtype, batch):
    """bf16 weights at batches 256 (the headline shape) and 128 (the first
    batch with the lo correction); e4m3 weights at batch 1024 (config 5: the
    256 bench positions four times over, each copy bit-equal).  Eager run,
    graph capture and two replays bit-equal; gates against the oracle on the
    same (dequantised) weights."""
    spec = synth.SPECS["bt4"]
    weights, planes, _, ref_all = bt4_bench_oracle(weights_dtype == "fp8")
    assert np.array_equal(planes, positions["planes"])
    n = min(batch, 256)
    ref = {k: v[:n] for k, v in ref_all.items()}
    idx = np.arange(batch) % n
    net = backend.create_network(spec, weights, max_batch=batch, device=0,
                                 weights_dtype=weights_dtype, precision="bf16x2_fp8lo")
    assert "bf16x2_fp8lo" in net.info(), net.info()
    runs = _device_runs(net, positions["masks"][idx], positions["values"][idx])
    net.close()
    for pol, wdl in runs[1:]:
        assert np.array_equal(_bits(pol), _bits(runs[0][0]))
        assert np.array_equal(_bits(wdl), _bits(runs[0][1]))
    pol, wdl = runs[-1]
    for r in range(1, batch // n):
        assert np.array_equal(_bits(pol[r * n:(r + 1) * n]), _bits(pol[:n])), r
    perr = float(np.abs(pol - ref["policy"][idx]).max())
    werr = float(np.abs(wdl - ref["wdl"][idx]).max())
    top1 = _top1(pol, ref["policy"][idx], positions["legal"][idx])
    print(f"bf16x2_fp8lo, {weights_dtype} weights, batch {batch}: policy max-abs {perr:.3e} "
          f"wdl max-abs {werr:.3e} top-1 {top1:.4f}", flush=True)
    assert perr <= POLICY_TOL and werr <= WDL_TOL and top1 >= TOP1_GATE


def test_widths_not_multiple_of_128_rejected():
    """The lo pass takes 128-byte K steps: a net whose FFN width is not a
    multiple of 128 is refused at creation, not at its first forward (the
    embedding width, 32 per head and heads a multiple of 4, always is)."""
    spec = synth.NetSpec("ffn448", 256, 1, 8, 448, input_ffn=512, policy_dim=256)
    weights = synth.make_weights(spec, seed=0)
    with pytest.raises(RuntimeError, match="multiples of 128"):
        backend.create_network(spec, weights, max_batch=8, device=0, precision="bf16x2_fp8lo")
    net = backend.create_network(spec, weights, max_batch=8, device=0, precision="bf16x2")
    net.close()
