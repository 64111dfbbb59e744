"""The C++ NN::Network adapter (HipNetwork over the C ABI), driven by
metalfish_amd/hip_network_test: EvaluateBatch with chunking past max_batch,
Evaluate per position, capabilities, and the exception path.

The driver reads the net and planes from files this test writes and returns
the decoded NetworkOutput fields (policy, WDL, value = W - L)."""

import os
import struct
import subprocess

import numpy as np
import pytest

import netfile
import oracle
from metalfish_amd import backend, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "metalfish_amd", "hip_network_test")


def _write_net(path, weights):
    with open(path, "wb") as f:
        f.write(struct.pack("<I", len(weights)))
        for name, arr in weights.items():
            raw = name.encode()
            data = np.ascontiguousarray(arr, dtype=np.float32).reshape(-1)
            f.write(struct.pack("<I", len(raw)) + raw + struct.pack("<Q", data.size))
            f.write(data.tobytes())


def _write_planes(path, planes):
    with open(path, "wb") as f:
        f.write(struct.pack("<I", planes.shape[0]))
        f.write(np.ascontiguousarray(planes, dtype=np.float32).tobytes())


def _run(tmp_path, weights, planes, heads, precision="bf16x2", max_batch=8):
    net, pl, out = (str(tmp_path / n) for n in ("net.bin", "planes.bin", "out.bin"))
    _write_net(net, weights)
    _write_planes(pl, planes)
    proc = subprocess.run([DRIVER, net, pl, out, str(heads), precision, str(max_batch)],
                          capture_output=True, text=True, timeout=300)
    return proc, out


@pytest.fixture(scope="module")
def plumbing():
    spec = synth.SPECS["cpu_plumbing"]
    return spec, synth.make_weights(spec, seed=3)


def test_driver_built():
    assert os.access(DRIVER, os.X_OK), "run __graft_entry__.build() first"


def test_adapter_throws_cleanly_without_a_device(tmp_path, plumbing):
    if backend.device_count() > 0:
        pytest.skip("a GPU is visible")
    spec, weights = plumbing
    planes, _ = synth.playout_positions(2, seed=1)
    proc, _ = _run(tmp_path, weights, planes, spec.heads)
    # std::runtime_error from the constructor, caught by the driver (exit 3).
    assert proc.returncode == 3, proc.stderr
    assert "HIP backend initialisation failed" in proc.stderr


@pytest.mark.gpu
def test_adapter_matches_oracle_with_chunking(tmp_path, plumbing):
    spec, weights = plumbing
    n = 20  # max_batch 8: chunks of 8, 8, 4
    planes, legal = synth.playout_positions(n, seed=9)
    proc, out = _run(tmp_path, weights, planes, spec.heads)
    assert proc.returncode == 0, proc.stderr
    got = np.fromfile(out, dtype=np.float32).reshape(2, n, 1858 + 4)
    # EvaluateBatch and per-position Evaluate give the same bits (batch
    # invariance), so the chunk boundaries leave no trace.
    assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32))
    ref = oracle.OracleNet(oracle.NetFormat(body_heads=spec.heads), weights).evaluate_batch(planes)
    policy, wdl, value = got[0, :, :1858], got[0, :, 1858:1861], got[0, :, 1861]
    assert np.abs(policy - ref["policy"]).max() <= 2e-2
    assert np.abs(wdl - ref["wdl"]).max() <= 5e-3
    assert np.array_equal(value, wdl[:, 0] - wdl[:, 2])


def _write_pb(path, spec, weights):
    netfile.write(path, netfile.spec_net_bytes(spec, weights, synth.tensor_layout(spec)))


def test_adapter_file_errors_without_a_device(tmp_path, plumbing):
    spec, weights = plumbing
    planes, _ = synth.playout_positions(2, seed=1)
    pl, out = str(tmp_path / "planes.bin"), str(tmp_path / "out.bin")
    _write_planes(pl, planes)
    bad = tmp_path / "bad.pb"
    bad.write_bytes(b"\x0d\x00\x00\x00\x00")
    proc = subprocess.run([DRIVER, str(bad), pl, out, "0", "bf16x2", "8"], capture_output=True,
                          text=True, timeout=300)
    assert proc.returncode == 3 and "bad magic number" in proc.stderr, proc.stderr
    good = tmp_path / "net.pb.gz"
    _write_pb(good, spec, weights)
    # The factory serves "hip", "auto" and "accelerator" only.
    proc = subprocess.run([DRIVER, str(good), pl, out, "0", "bf16x2", "8"], capture_output=True,
                          text=True, timeout=300, env={**os.environ, "MFH_TEST_BACKEND": "cuda"})
    assert proc.returncode == 3 and 'cannot serve backend "cuda"' in proc.stderr, proc.stderr
    if backend.device_count() > 0:
        return
    proc = subprocess.run([DRIVER, str(good), pl, out, "0", "bf16x2", "8"], capture_output=True,
                          text=True, timeout=300)
    # The file loads; creating the net needs the device.
    assert proc.returncode == 3 and "HIP backend initialisation failed" in proc.stderr, \
        proc.stderr


@pytest.mark.gpu
def test_adapter_from_network_file_matches_tensors(tmp_path, plumbing):
    """HipNetwork(weights_path, config) on a .pb.gz of the net gives the same
    bits as HipNetwork(tensors, config)."""
    spec, weights = plumbing
    planes, _ = synth.playout_positions(12, seed=5)
    proc, out = _run(tmp_path, weights, planes, spec.heads)
    assert proc.returncode == 0, proc.stderr
    ref = np.fromfile(out, dtype=np.float32)
    net = str(tmp_path / "net.pb.gz")
    _write_pb(net, spec, weights)
    pl, out2 = str(tmp_path / "planes.bin"), str(tmp_path / "out2.bin")
    proc = subprocess.run([DRIVER, net, pl, out2, "0", "bf16x2", "8"], capture_output=True,
                          text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr
    assert np.array_equal(np.fromfile(out2, dtype=np.float32).view(np.uint32), ref.view(np.uint32))


@pytest.mark.gpu
def test_adapter_priors_match_cpu_computation(tmp_path, plumbing):
    """HipNetwork::EvaluateBatchPriors: per position, the priors of its legal
    moves equal the reference's CPU computation on the logits EvaluateBatch
    returns, bit for bit, across max_batch chunks."""
    spec, weights = plumbing
    n = 20
    planes, legal = synth.playout_positions(n, seed=21)
    moves = [l[l >= 0].astype(np.int16) for l in legal]
    offsets = np.zeros(n + 1, np.int32)
    offsets[1:] = np.cumsum([m.size for m in moves])
    mv = tmp_path / "moves.bin"
    mv.write_bytes(offsets.tobytes() + np.concatenate(moves).tobytes())
    net, pl, out = (str(tmp_path / x) for x in ("net.bin", "planes.bin", "out.bin"))
    _write_net(net, weights)
    _write_planes(pl, planes)
    proc = subprocess.run([DRIVER, net, pl, out, str(spec.heads), "bf16x2", "8", str(mv), "0.7"],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr
    got = np.fromfile(out, dtype=np.float32)
    base = got[:2 * n * (1858 + 4)].reshape(2, n, 1858 + 4)
    priors = got[2 * n * (1858 + 4):2 * n * (1858 + 4) + offsets[-1]]
    tail = got[2 * n * (1858 + 4) + offsets[-1]:].reshape(n, 4)
    for b in range(n):
        want = oracle.mcts_priors(base[0, b, :1858], moves[b], 0.7)
        assert np.array_equal(priors[offsets[b]:offsets[b + 1]].view(np.uint32),
                              want.view(np.uint32)), b
    assert np.array_equal(tail.view(np.uint32), base[0, :, 1858:].view(np.uint32))
