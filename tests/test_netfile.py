"""Network-file reader (C ABI mfh_weights_*, metalfish_amd/csrc/host/
weights_file.cpp) against fixtures made by libprotobuf from the reference's
schema (tests/golden/make_netfiles.py), plus round trips through the
test-side writer (tests/netfile.py), which is itself pinned byte for byte
against libprotobuf output.  No device needed."""

import gzip
import json
import os

import numpy as np
import pytest

import netfile
from metalfish_amd import backend, synth

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "netfiles")
EXPECTED = json.load(open(os.path.join(FIX, "expected.json")))
ARRAYS = np.load(os.path.join(FIX, "expected.npz"))
GOOD = sorted(k for k, v in EXPECTED["fixtures"].items() if "error" not in v)
BAD = sorted(k for k, v in EXPECTED["fixtures"].items() if "error" in v)
F32_EPS = float(np.finfo(np.float32).eps)


def check_against_expected(w, name):
    exp = EXPECTED["fixtures"][name]
    assert w.format == exp["format"]
    assert w.headcount == exp["headcount"]
    assert w.pol_headcount == exp["pol_headcount"]
    assert [[n, w.dims[n]] for n in w.tensors] == [[n, d] for n, d, _ in exp["tensors"]]
    for n, _, kind in exp["tensors"]:
        got = w.tensors[n].astype(np.float64)
        want = ARRAYS[f"{name}/{n}"]
        if kind == "exact":
            np.testing.assert_array_equal(got, want, err_msg=n)
        else:
            # LINEAR16 is three float32 operations on exact inputs, the
            # batch-norm fold four: a few ulp of the operands' scale.
            scale = np.maximum(np.abs(want), np.abs(want).max() if kind == "linear16" else 0)
            np.testing.assert_array_less(np.abs(got - want), 4 * F32_EPS * scale + 1e-30,
                                         err_msg=n)


@pytest.mark.parametrize("name", GOOD)
def test_fixture_decodes_as_reference(name):
    check_against_expected(backend.load_weights(os.path.join(FIX, name + ".pb")), name)


@pytest.mark.parametrize("name", BAD)
def test_fixture_errors_as_reference(name):
    with pytest.raises(RuntimeError) as e:
        backend.load_weights(os.path.join(FIX, name + ".pb"))
    assert e.value.args[0].endswith(EXPECTED["fixtures"][name]["error"])


def test_gzip_file_matches_plain():
    check_against_expected(backend.load_weights(os.path.join(FIX, "every_field.pb.gz")),
                           "every_field")


def test_minimal_reference_fixture_inventory():
    """The reference's minimal attention fixture inventories exactly three
    one-element tensors with dims "1" (reference tests/test_mcts_module.cpp:
    115-140, 1561-1597)."""
    w = backend.load_weights(os.path.join(FIX, "minimal.pb"))
    assert list(w.tensors) == ["policy.vanilla.ip_pol_w", "value.winner.ip_val_w",
                               "moves_left.weights"]
    assert all(d == [1] for d in w.dims.values())
    assert sum(t.size for t in w.tensors.values()) == 3
    # DescribeNetworkFormat on the same fixture (test_mcts_module.cpp:1415-1436).
    assert w.format["input_embedding"] == 2 and w.format["ffn_activation"] == 7
    assert w.headcount == 0 and w.pol_headcount == 0


def test_parse_from_memory_matches_file():
    data = open(os.path.join(FIX, "every_field.pb"), "rb").read()
    check_against_expected(backend.parse_weights(data), "every_field")


@pytest.mark.parametrize("name", sorted(EXPECTED["writer"]))
def test_writer_is_byte_identical_to_libprotobuf(name):
    spec = EXPECTED["writer"][name]
    tensors = {n: ARRAYS[f"{name}/{n}"] for n, _, _ in spec["tensors"]}
    data = netfile.net_bytes(tensors, spec["format"], spec["headcount"], spec["pol_headcount"],
                             {n: e for n, e, _ in spec["tensors"]}, spec["legacy"],
                             dims={n: d for n, _, d in spec["tensors"]})
    assert data == open(os.path.join(FIX, name + ".pb"), "rb").read()


def test_fp16_decoding_every_code():
    """FLOAT16 widening is exact for all 65536 codes, subnormals, infinities
    and NaN payloads included (numpy's IEEE conversion as the check)."""
    codes = np.arange(65536, dtype=np.uint16)
    half = codes.view(np.float16)
    data = netfile.f_fixed32(1, 0x1C0) + netfile.f_bytes(10, netfile.f_bytes(
        45, netfile.f_bytes(3, netfile.f_bytes(1, netfile.f_bytes(3, codes.astype("<u2").tobytes())
                                               + netfile.f_varint(4, 2))))
        + netfile.f_bytes(29, netfile.f_bytes(3, b"\0\0\x80?") + netfile.f_varint(4, 4)))
    got = backend.parse_weights(data).tensors["policy.vanilla.ip_pol_w"]
    want = half.astype(np.float32)
    finite = np.isfinite(want)
    np.testing.assert_array_equal(got.view(np.uint32)[finite], want.view(np.uint32)[finite])
    # Inf and NaN keep sign and payload (fraction shifted into the top bits).
    nonfinite = ~finite
    exp_bits = ((codes[nonfinite].astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | \
        ((codes[nonfinite].astype(np.uint32) & 0x3FF) << 13)
    np.testing.assert_array_equal(got.view(np.uint32)[nonfinite], exp_bits)


def test_bf16_and_linear16_closed_forms():
    """BFLOAT16 is the top half of the binary32 pattern; LINEAR16 maps code 0
    to min exactly and every code q to min + q/65535*(max - min) within float32
    rounding."""
    codes = np.arange(0, 65536, 7, dtype=np.uint16)
    lo, hi = np.float32(-3.25), np.float32(1.5)
    ip = netfile.f_bytes(3, netfile.f_bytes(1, netfile.f_bytes(3, codes.astype("<u2").tobytes())
                                            + netfile.f_varint(4, 3)))
    lin = netfile.f_bytes(1, netfile.f_bytes(1, netfile.f_float(1, lo) + netfile.f_float(2, hi)
                                             + netfile.f_bytes(3, codes.astype("<u2").tobytes())))
    data = netfile.f_fixed32(1, 0x1C0) + netfile.f_bytes(10, netfile.f_bytes(44, lin)
                                                         + netfile.f_bytes(45, ip))
    w = backend.parse_weights(data)
    np.testing.assert_array_equal(w.tensors["policy.vanilla.ip_pol_w"].view(np.uint32),
                                  codes.astype(np.uint32) << 16)
    v = w.tensors["value.winner.ip_val_w"].astype(np.float64)
    assert v[0] == lo
    want = float(lo) + codes / 65535.0 * (float(hi) - float(lo))
    assert np.abs(v - want).max() <= 4 * F32_EPS * (abs(float(lo)) + abs(float(hi)))


def test_proto2_merge_and_unknown_fields():
    """Repeated occurrences of a message merge, the last scalar wins, unknown
    fields (any wire type, groups included) are skipped, a known field with
    the wrong wire type is ignored, packed dims are accepted, and an enum
    value outside the enum leaves the field unset."""
    one = netfile.f_bytes(3, np.float32([1.0]).tobytes()) + netfile.f_varint(4, 4)
    two = netfile.f_bytes(3, np.float32([2.0, 3.0]).tobytes()) + netfile.f_varint(4, 4)
    unknown = (netfile.f_varint(999, 5) + netfile.f_fixed32(998, 7) + netfile._key(997, 1)
               + b"\0" * 8 + netfile._key(996, 3) + netfile.f_varint(1, 1) + netfile._key(996, 4)
               + netfile.f_bytes(995, b"xyz"))
    packed_dims = netfile.f_bytes(5, netfile._varint(1) + netfile._varint(2))
    heads = netfile.f_bytes(3, netfile.f_bytes(1, one) + unknown)      # vanilla, part 1
    heads += netfile.f_bytes(3, netfile.f_bytes(3, two + packed_dims))  # vanilla, part 2
    weights = netfile.f_bytes(45, heads) + netfile.f_bytes(29, one)
    weights += netfile.f_varint(28, 3) + netfile.f_varint(28, 5)        # headcount: last wins
    weights += netfile.f_fixed32(25, 0)                                   # ip_emb_w, wrong wire
    nf = netfile.f_varint(3, 7) + netfile.f_varint(5, 2) + netfile.f_varint(5, 77)
    data = (netfile.f_fixed32(1, 0x1C0) + netfile.f_bytes(4, netfile.f_bytes(2, nf))
            + unknown + netfile.f_bytes(10, weights))
    w = backend.parse_weights(data)
    assert w.headcount == 5
    assert w.format["value"] == 2  # 77 is not a ValueFormat
    np.testing.assert_array_equal(w.tensors["policy.vanilla.ip_pol_w"], [1.0])
    np.testing.assert_array_equal(w.tensors["policy.vanilla.ip2_pol_w"], [2.0, 3.0])
    assert w.dims["policy.vanilla.ip2_pol_w"] == [1, 2]
    assert "body.ip_emb_w" not in w.tensors


def test_malformed_wire_data_is_rejected():
    good = netfile.f_fixed32(1, 0x1C0) + netfile.f_bytes(10, netfile.f_bytes(
        4, netfile.f_bytes(3, b"\0\0\x80?")) + netfile.f_bytes(29, netfile.f_bytes(3, b"\0" * 4)))
    backend.parse_weights(good)
    for bad in (good + b"\x80",                       # truncated varint key
                good + netfile._key(7, 6),            # reserved wire type
                good + netfile._key(7, 4),            # stray end-group
                good + netfile._key(7, 2) + b"\x05ab",  # length past the end
                good + b"\x00\x00",                   # field number 0
                good + b"\xff" * 11):                 # overlong varint
        with pytest.raises(RuntimeError, match="Failed to parse protobuf weights file"):
            backend.parse_weights(bad)


@pytest.mark.parametrize("encoding", ["f32", "f16", "bf16", "linear16"])
def test_round_trip_cpu_plumbing_net(tmp_path, encoding):
    """A whole benchmark-shape net written with each encoding reads back as
    the same inventory (values exact up to the encoding's own rounding)."""
    spec = synth.SPECS["cpu_plumbing"]
    weights = synth.make_weights(spec, seed=3)
    fmt = dict(network=7, policy=3, value=2, input_embedding=2, default_activation=1,
               smolgen_activation=7, ffn_activation=0)
    path = tmp_path / ("net.pb.gz" if encoding == "bf16" else "net.pb")
    netfile.write(path, netfile.net_bytes(weights, fmt, spec.heads, encoding=encoding,
                                          dims={n: list(a.shape) for n, a in weights.items()}))
    w = backend.load_weights(str(path))
    assert list(w.tensors) == list(weights)
    assert w.headcount == spec.heads
    for n, a in weights.items():
        assert w.dims[n] == list(a.shape)
        want = netfile.decoded(a, encoding)
        if encoding == "linear16":
            lo, hi = float(a.min()), float(a.max())
            assert np.abs(w.tensors[n] - a.reshape(-1)).max() <= (hi - lo) / 65535 * 0.5 + \
                4 * F32_EPS * max(abs(lo), abs(hi)), n
            np.testing.assert_allclose(w.tensors[n], want, rtol=0,
                                       atol=4 * F32_EPS * max(abs(lo), abs(hi)), err_msg=n)
        else:
            np.testing.assert_array_equal(w.tensors[n], want, err_msg=n)


def test_legacy_head_fields_round_trip():
    spec = synth.SPECS["cpu_plumbing"]
    weights = synth.make_weights(spec, seed=4)
    data = netfile.net_bytes(weights, dict(network=6, policy=3, value=2), spec.heads,
                             legacy_heads=True)
    w = backend.parse_weights(data)
    assert list(w.tensors) == list(weights)
    # Attention body with head format and no input_embedding: PE_MAP.
    assert w.format["network"] == 6 and w.format["input_embedding"] == 1
    for n, a in weights.items():
        np.testing.assert_array_equal(w.tensors[n], a.reshape(-1))


def test_gzip_reader_handles_multi_member_and_plain_bytes(tmp_path):
    """zlib's reader concatenates gzip members and passes non-gzip bytes
    through, as the reference's gzread loop does."""
    data = open(os.path.join(FIX, "every_field.pb"), "rb").read()
    p = tmp_path / "two_members.pb.gz"
    with open(p, "wb") as f:
        f.write(gzip.compress(data[:1000]) + gzip.compress(data[1000:]))
    check_against_expected(backend.load_weights(str(p)), "every_field")
    p = tmp_path / "plain.pb.gz"
    p.write_bytes(data)
    check_against_expected(backend.load_weights(str(p)), "every_field")


def test_missing_file_errors():
    with pytest.raises(RuntimeError, match="Cannot read weights from"):
        backend.load_weights("/nonexistent/net.pb")
    with pytest.raises(RuntimeError, match="Cannot read weights from"):
        backend.load_weights("/nonexistent/net.pb.gz")
