"""The C ABI libraries load, export every function their headers declare,
and reject bad input with a status and message, without a GPU."""

import ctypes
import os
import re

import numpy as np
import pytest

from metalfish_amd import backend, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    return sorted(set(re.findall(r"\b(mf[hs]_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("mfhip.h", "libmfhip.so"),
                                        ("mfh_synth.h", "libmfhost.so")])
def test_exports_match_header(header, lib):
    names = declared(header)
    assert names
    so = ctypes.CDLL(os.path.join(ROOT, "metalfish_amd", lib))
    for name in names:
        assert hasattr(so, name), f"{lib} lacks {name}"


def test_python_binding_covers_header():
    assert sorted(backend.EXPORTS) == declared("mfhip.h")


def _desc(**kw):
    d = dict(network=6, policy=3, value=2, moves_left=0, input_embedding=2,
             default_activation=1, ffn_activation=0, smolgen_activation=7, headcount=8,
             weights_dtype=0, precision=1, max_batch=4, device=-1)
    d.update(kw)
    return backend.MfhNetDesc(**d)


def _create(desc, weights):
    names = list(weights)
    keep = [np.ascontiguousarray(weights[n], dtype=np.float32).reshape(-1) for n in names]
    enc = [n.encode() for n in names]
    tensors = (backend.MfhTensor * len(names))(
        *[backend.MfhTensor(enc[i], keep[i].ctypes.data, keep[i].size) for i in range(len(names))])
    handle = ctypes.c_void_p()
    rc = backend.lib().mfh_net_create(ctypes.byref(desc), tensors, len(names), ctypes.byref(handle))
    return rc, backend.lib().mfh_last_error().decode()


def test_unsupported_structures_are_rejected_before_touching_a_device():
    w = synth.make_weights(synth.SPECS["cpu_plumbing"], seed=0)
    # PE_MAP declared for a net with dynamic-PE weights and a 112 + 16 input.
    rc, msg = _create(_desc(input_embedding=1), w)
    assert rc == -3 and "PE_MAP" in msg
    rc, msg = _create(_desc(input_embedding=0), w)
    assert rc == -3 and "input embeddings" in msg
    # Moves-left head declared without its tensors.
    rc, msg = _create(_desc(moves_left=1), w)
    assert rc == -3 and "moves-left" in msg
    rc, msg = _create(_desc(moves_left=2), w)
    assert rc == -3 and "moves-left" in msg
    rc, msg = _create(_desc(headcount=4), w)  # head depth 64
    assert rc == -3 and "head depth" in msg
    bad = dict(w)
    del bad["body.encoder.0.ffn.dense1_w"]
    rc, msg = _create(_desc(), bad)
    assert rc in (-1, -4)  # missing tensor (or no device, checked after shapes)


def test_device_count_without_gpu_is_zero_or_more():
    assert backend.device_count() >= 0


def test_pack_planes_rejects_null():
    assert backend.lib().mfh_pack_planes(2, None, None, None) == -1
