"""mfh_net_eval_device_noalloc: the forward with its workspace in the
library's static scratch array, for callers that cannot allocate device
memory.  Checked against mfh_net_eval_device (the existing device entry
point, same kernels) bit for bit on two calls in a row, the second with a
smaller batch; after another net has used the array in between (the array
is shared per device and keeps the last call's contents); and batches beyond
the reported limit are rejected."""

import re

import numpy as np
import pytest

import gpu_util
from metalfish_amd import backend, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if backend.device_count() < 1:
        pytest.fail("GPU tests need an MI355X; none visible")


def _limit(net):
    m = re.search(r"no-allocation batch <= (\d+)", net.info())
    assert m, net.info()
    return int(m.group(1))


def _call(net, entry, dev, stream, batch, d_m, d_v):
    pol = np.full((batch, 1858), np.nan, np.float32)
    wdl = np.full((batch, 3), np.nan, np.float32)
    d_p, d_w = dev.put(pol), dev.put(wdl)
    rc = getattr(backend.lib(), entry)(net._h, batch, d_m, d_v, d_p, d_w, stream)
    assert rc == backend.MFH_OK, backend.lib().mfh_last_error()
    dev.sync(stream)
    return dev.get(d_p, pol), dev.get(d_w, wdl)


def _same(a, b):
    return all(np.array_equal(np.ascontiguousarray(x).view(np.uint32),
                              np.ascontiguousarray(y).view(np.uint32)) for x, y in zip(a, b))


@pytest.mark.parametrize("spec_name,precision,limit", [
    ("cpu_plumbing", "bf16x2", 31), ("bt4", "bf16x2", 15), ("bt4", "bf16", 27)])
def test_noalloc_entry_matches_eval_device(spec_name, precision, limit):
    spec = synth.SPECS[spec_name]
    weights = synth.make_weights(spec, seed=0)
    planes, _ = synth.playout_positions(40, seed=21)
    masks, values = backend.pack_planes(planes)
    net = backend.create_network(spec, weights, max_batch=32, device=0, precision=precision)
    assert _limit(net) == limit
    other_spec = synth.SPECS["cpu_plumbing"]
    other = backend.create_network(other_spec, synth.make_weights(other_spec, seed=1),
                                   max_batch=8, device=0)
    dev = gpu_util.DeviceBuffers()
    stream = dev.stream()
    cases = [(limit, 0), (3, 30)]  # the second call is smaller (other positions)
    inputs = [(dev.put(masks[s:s + b]), dev.put(values[s:s + b])) for b, s in cases]
    want = [_call(net, "mfh_net_eval_device", dev, stream, b, *io)
            for (b, _), io in zip(cases, inputs)]
    print(f"{spec_name} {precision}: no-allocation limit {limit}; {net.info()}", flush=True)
    for k in range(2):  # two calls in a row, larger then smaller
        got = _call(net, "mfh_net_eval_device_noalloc", dev, stream, cases[k][0], *inputs[k])
        assert _same(got, want[k]), (spec_name, precision, cases[k])
    # Another net uses the shared array, then this net again (smaller batch).
    o_m, o_v = dev.put(masks[:8]), dev.put(values[:8])
    o_want = _call(other, "mfh_net_eval_device", dev, stream, 8, o_m, o_v)
    assert _same(_call(other, "mfh_net_eval_device_noalloc", dev, stream, 8, o_m, o_v), o_want)
    got = _call(net, "mfh_net_eval_device_noalloc", dev, stream, cases[1][0], *inputs[1])
    assert _same(got, want[1])
    # Beyond the limit (and batch 0): rejected before any device work.
    lib = backend.lib()
    for bad in (limit + 1, 0):
        rc = lib.mfh_net_eval_device_noalloc(net._h, bad, inputs[0][0], inputs[0][1],
                                             inputs[0][0], inputs[0][1], stream)
        assert rc == -1 and b"scratch array" in lib.mfh_last_error(), bad
    dev.free()
    other.close()
    net.close()
