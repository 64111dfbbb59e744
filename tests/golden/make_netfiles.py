"""Writes the network-file fixtures under tests/golden/netfiles/ (run in the
build container, where the reference tree and a protoc binary exist).

The files are made by libprotobuf itself (the Python runtime), from the
reference's own schema (reference src/nn/proto/net.proto, compiled to a
descriptor set by the protoc that ships with torch), with fields set by their
schema names, so they pin both this repository's proto2 reader
(metalfish_amd/csrc/host/weights_file.cpp) and its test-side writer
(tests/netfile.py) independently of the field numbers either one restates.

expected.json holds, per fixture, what the reference's loader makes of the
file: the NetworkFormat after FixOlderWeightsFile (reference
src/nn/loader.cpp:86-135, PE_MAP default network_format.cpp:97-100), the
head counts, and the inventory of the selected heads in the reference's
order (network_weight_inventory.cpp:116-352) with dims; or the error message
the reference throws.  expected.npz holds the decoded values
("<fixture>/<tensor>"): exact source values for FLOAT32/FLOAT16/BFLOAT16
layers (the sources are chosen representable), float64 evaluations of the
LINEAR16 definition and of the batch-norm fold (weights.cpp:91-143) for the
others -- the test compares those within a few ulp.

Usage: python tests/golden/make_netfiles.py
"""

import gzip
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "netfiles")
PROTO_DIR = "/root/reference/src/nn/proto"
PROTOC = os.path.join(os.path.dirname(__import__("torch").__file__), "bin", "protoc")

from google.protobuf import descriptor_pb2, descriptor_pool, message_factory  # noqa: E402


def load_schema():
    with tempfile.TemporaryDirectory() as tmp:
        out = os.path.join(tmp, "net.desc")
        subprocess.run([PROTOC, f"--proto_path={PROTO_DIR}", f"--descriptor_set_out={out}",
                        "net.proto"], check=True)
        fds = descriptor_pb2.FileDescriptorSet.FromString(open(out, "rb").read())
    pool = descriptor_pool.DescriptorPool()
    for f in fds.file:
        pool.Add(f)
    pkg = fds.file[0].package
    return message_factory.GetMessageClass(pool.FindMessageTypeByName(pkg + ".Net"))


Net = load_schema()
LAYER_ENCODING = {"linear16": 1, "f16": 2, "bf16": 3, "f32": 4}
rng = np.random.default_rng(20251201)


def values_for(encoding, n):
    """Source values representable in the encoding."""
    v = rng.standard_normal(n).astype(np.float32)
    if encoding == "f16":
        v = v.astype(np.float16).astype(np.float32)
    elif encoding == "bf16":
        v = (v.view(np.uint32) & 0xFFFF0000).view(np.float32)
    return v


def set_layer(layer, values, encoding, dims=None):
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    if encoding in ("linear16", "unset"):
        lo, hi = float(v.min()), float(v.max())
        q = np.rint((v.astype(np.float64) - lo) / (hi - lo) * 65535.0).astype(np.uint16)
        layer.min_val = lo
        layer.max_val = hi
        layer.params = q.astype("<u2").tobytes()
    elif encoding == "f16":
        layer.params = v.astype("<f2").tobytes()
    elif encoding == "bf16":
        layer.params = (v.view(np.uint32) >> 16).astype("<u2").tobytes()
    else:
        layer.params = v.astype("<f4").tobytes()
    if encoding != "unset":
        layer.encoding = LAYER_ENCODING[encoding]
    for d in (dims if dims is not None else [v.size]):
        layer.dims.append(int(d))


def decoded(values, encoding):
    """Float64 view of what the layer holds after decoding."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    if encoding in ("linear16", "unset"):
        lo, hi = np.float32(v.min()), np.float32(v.max())
        q = np.rint((v.astype(np.float64) - float(lo)) / (float(hi) - float(lo)) * 65535.0)
        return float(lo) + q / 65535.0 * (float(hi) - float(lo))
    return v.astype(np.float64)


def resolve(msg, path):
    """Walks schema attribute names; integer parts index repeated fields."""
    for part in path:
        if isinstance(part, int):
            while len(msg) <= part:
                msg.add()
            msg = msg[part]
        else:
            msg = getattr(msg, part)
    return msg


def attr_path(name, legacy):
    """Inventory name -> schema attribute path (the inventory names are the
    schema's field names, network_weight_inventory.cpp:37-180)."""
    parts = [int(p) if p.isdigit() else p for p in name.split(".")]
    if parts[0] == "body":
        return ["weights"] + parts[1:]
    if parts[0] == "moves_left":
        return ["weights"] + (["moves_left", parts[1]] if parts[1] in CONV_FIELDS else [parts[1]])
    rest = parts[2:]
    if rest[0] == "encoder":
        rest = ["pol_encoder"] + rest[1:]
    if parts[0] == "policy":
        return ["weights"] + (rest if legacy else ["policy_heads", parts[1]] + rest)
    return ["weights"] + (rest if legacy else ["value_heads", parts[1]] + rest)


CONV_FIELDS = ("weights", "biases", "bn_means", "bn_stddivs", "bn_gammas", "bn_betas")


class Fixture:
    def __init__(self, name, legacy=False):
        self.name = name
        self.legacy = legacy
        self.net = Net()
        self.net.magic = 0x1C0
        self.expected = []  # (inventory name, dims, float64 values, kind)

    def fmt(self, **fields):
        nf = self.net.format.network_format
        for k, v in fields.items():
            setattr(nf, k, v)

    def tensor(self, name, n=4, encoding="f32", dims=None, expect=True):
        v = values_for("f32" if encoding in ("linear16", "unset") else encoding, n)
        set_layer(resolve(self.net, attr_path(name, self.legacy)), v, encoding, dims)
        if expect:
            kind = "linear16" if encoding in ("linear16", "unset") else "exact"
            self.expected.append((name, list(dims) if dims else [n], decoded(v, encoding), kind))
        return v

    def conv(self, prefix, outputs=2, inputs=3, bn=("means", "stddivs", "gammas", "betas"),
             biases=True):
        """A ConvBlock (f32 layers) and its folded inventory entries
        (BaseWeights::ConvBlock, weights.cpp:91-143, evaluated in float64)."""
        path = attr_path(prefix + ".weights", self.legacy)[:-1]
        block = resolve(self.net, path)
        w = values_for("f32", outputs * inputs)
        set_layer(block.weights, w, "f32", [outputs, inputs])
        b = values_for("f32", outputs) if biases else None
        if biases:
            set_layer(block.biases, b, "f32")
        parts = {}
        for f in bn:
            v = values_for("f32", outputs)
            if f == "stddivs":
                v = np.abs(v) + np.float32(0.5)
            parts[f] = v
            set_layer(getattr(block, "bn_" + f), v, "f32")
        w64 = w.astype(np.float64).reshape(outputs, inputs)
        b64 = b.astype(np.float64) if biases else np.zeros(outputs)
        if "means" in parts:
            # Missing betas: betas 0 and gammas 1 are appended per mean.
            gam = parts["gammas"].astype(np.float64) if "gammas" in parts else np.ones(outputs)
            bet = parts["betas"].astype(np.float64) if "betas" in parts else np.zeros(outputs)
            sd = parts["stddivs"].astype(np.float64)
            g = gam / np.sqrt(sd + float(np.float32(1e-5)))
            folded_w = w64 * g[:, None]
            folded_b = bet - g * (parts["means"].astype(np.float64) - b64)
            self.expected.append((prefix + ".weights", [outputs, inputs], folded_w.reshape(-1),
                                  "bnfold"))
            self.expected.append((prefix + ".biases", [outputs], folded_b, "bnfold"))
        else:
            self.expected.append((prefix + ".weights", [outputs, inputs], w64.reshape(-1),
                                  "exact"))
            if biases:
                self.expected.append((prefix + ".biases", [outputs], b64, "exact"))

    def encoder(self, prefix, smolgen=True, encodings=("f32",)):
        names = [f"{prefix}.mha.{t}" for t in ("q_w", "q_b", "k_w", "k_b", "v_w", "v_b",
                                                 "dense_w", "dense_b")]
        if smolgen:
            names += [f"{prefix}.mha.smolgen.{t}" for t in (
                "compress", "dense1_w", "dense1_b", "ln1_gammas", "ln1_betas", "dense2_w",
                "dense2_b", "ln2_gammas", "ln2_betas")]
        names += [f"{prefix}.ln1_gammas", f"{prefix}.ln1_betas"]
        names += [f"{prefix}.ffn.{t}" for t in ("dense1_w", "dense1_b", "dense2_w", "dense2_b")]
        names += [f"{prefix}.ln2_gammas", f"{prefix}.ln2_betas"]
        for i, n in enumerate(names):
            self.tensor(n, 3 + i % 3, encodings[i % len(encodings)])


BODY_EMBED = ["ip_emb_preproc_w", "ip_emb_preproc_b", "ip_emb_w", "ip_emb_b", "ip_emb_ln_gammas",
              "ip_emb_ln_betas", "ip_mult_gate", "ip_add_gate"]
ALL_ENC = ("f32", "f16", "bf16", "linear16", "unset")


def body(fx, encoder_layers=1, smolgen=True, residual=False, input_conv=False):
    if input_conv:
        fx.conv("body.input")
    for i, n in enumerate(BODY_EMBED):
        dims = [2, 3] if n == "ip_emb_w" else None
        fx.tensor("body." + n, 6 if dims else 4 + i % 2, ALL_ENC[i % 5], dims)
    for i, t in enumerate(("dense1_w", "dense1_b", "dense2_w", "dense2_b")):
        fx.tensor("body.ip_emb_ffn." + t, 3, ALL_ENC[(i + 2) % 5])
    fx.tensor("body.ip_emb_ffn_ln_gammas", 4, "f16")
    fx.tensor("body.ip_emb_ffn_ln_betas", 4, "bf16")
    if smolgen:
        fx.tensor("body.smolgen_w", 8, "linear16", [2, 4])
    for i in range(encoder_layers):
        fx.encoder(f"body.encoder.{i}", smolgen=smolgen, encodings=ALL_ENC)
    if residual:
        fx.conv("body.residual.0.conv1", biases=False)
        fx.conv("body.residual.0.conv2", bn=("means", "stddivs"))
        for t in ("w1", "b1", "w2", "b2"):
            fx.tensor("body.residual.0.se." + t, 2)


def policy(fx, encoder_layers=0, conv=False, skip_ip=False):
    h = "policy.vanilla."
    if conv:
        fx.conv(h + "policy1", bn=())
        fx.conv(h + "policy")
    names = ["ip_pol_w", "ip_pol_b", "ip2_pol_w", "ip2_pol_b", "ip3_pol_w", "ip3_pol_b",
             "ip4_pol_w"]
    for i, n in enumerate(names):
        if skip_ip and n in ("ip_pol_w", "ip_pol_b"):
            continue
        fx.tensor(h + n, 4, ALL_ENC[(i + 1) % 5])
    for i in range(encoder_layers):
        fx.encoder(f"{h}encoder.{i}", smolgen=False)


def value(fx, conv=False, err=False):
    h = "value.winner."
    if conv:
        fx.conv(h + "value")
    for i, n in enumerate(("ip_val_w", "ip_val_b", "ip1_val_w", "ip1_val_b", "ip2_val_w",
                           "ip2_val_b")):
        fx.tensor(h + n, 3, ALL_ENC[(i + 3) % 5])
    if err:
        fx.tensor(h + "ip_val_err_w", 2)
        fx.tensor(h + "ip_val_err_b", 1)


def moves_left(fx):
    fx.conv("moves_left", bn=("means", "stddivs", "gammas", "betas"))
    for n in ("ip_mov_w", "ip_mov_b", "ip1_mov_w", "ip1_mov_b", "ip2_mov_w", "ip2_mov_b"):
        fx.tensor("moves_left." + n, 2)


FORMAT_KEYS = ("input", "output", "network", "policy", "value", "moves_left",
               "default_activation", "smolgen_activation", "ffn_activation", "input_embedding")


def format_dict(**kw):
    d = {k: 0 for k in FORMAT_KEYS}
    d.update(kw)
    return d


def build():
    fixtures = []  # (Fixture, expected format, headcount, pol_headcount, sort_key)

    # The reference's minimal attention fixture (test_mcts_module.cpp:115-140),
    # whose inventory is exactly three one-element tensors (1561-1597).
    fx = Fixture("minimal")
    fx.fmt(network=7, policy=3, value=2, moves_left=1, input_embedding=2, default_activation=1,
           smolgen_activation=0, ffn_activation=7)
    for n in ("policy.vanilla.ip_pol_w", "value.winner.ip_val_w", "moves_left.weights"):
        layer = resolve(fx.net, attr_path(n, False))
        set_layer(layer, np.ones(1, np.float32), "f32", [1])
        fx.expected.append((n, [1], np.ones(1), "exact"))
    fixtures.append((fx, format_dict(network=7, policy=3, value=2, moves_left=1,
                                     input_embedding=2, default_activation=1,
                                     ffn_activation=7), 0, 0))

    # Every field of a multi-head attention net in every encoding, with
    # convolution blocks (batch norm folded), an SE unit, policy encoder
    # layers and the moves-left head.
    fx = Fixture("every_field")
    fx.fmt(input=5, output=2, network=7, policy=3, value=2, moves_left=1, default_activation=1,
           smolgen_activation=7, ffn_activation=1, input_embedding=2)
    fx.net.weights.headcount = 4
    body(fx, encoder_layers=2, residual=True, input_conv=True)
    policy(fx, encoder_layers=1, conv=True)
    fx.net.weights.policy_heads.vanilla.pol_headcount = 2
    value(fx, conv=True, err=True)
    moves_left(fx)
    # Heads that are not selected are not in the inventory.
    set_layer(fx.net.weights.policy_heads.optimistic_st.ip2_pol_w, np.ones(2, np.float32), "f32")
    set_layer(fx.net.weights.value_heads.q.ip_val_w, np.ones(2, np.float32), "f32")
    # Other top-level messages are parsed and ignored.
    fx.net.license = "test fixture"
    fx.net.min_version.major = 0
    fx.net.min_version.minor = 31
    fx.net.training_params.training_steps = 12345
    # Inventory order: body.input first (network_weight_inventory.cpp:118).
    order = ["body.input.weights", "body.input.biases"]
    fx.expected.sort(key=lambda e: order.index(e[0]) if e[0] in order else 2)
    fixtures.append((fx, format_dict(input=5, output=2, network=7, policy=3, value=2, moves_left=1,
                                     default_activation=1, smolgen_activation=7, ffn_activation=1,
                                     input_embedding=2), 4, 2))

    # Shared policy embedding (PolicyHeads.ip_pol_w/b, weights.cpp:216-226),
    # and ATTENTIONBODY_WITH_HEADFORMAT with both head messages -> multi-head
    # format with PE_DENSE (loader.cpp:124-134).
    fx = Fixture("shared_policy_embedding")
    fx.fmt(network=6, policy=3, value=2, default_activation=1)
    fx.net.weights.headcount = 2
    body(fx, encoder_layers=1, smolgen=False)
    w = values_for("f16", 4)
    set_layer(fx.net.weights.policy_heads.ip_pol_w, w, "f16")
    b = values_for("bf16", 2)
    set_layer(fx.net.weights.policy_heads.ip_pol_b, b, "bf16")
    n_before = len(fx.expected)
    policy(fx, skip_ip=True)
    fx.expected.insert(n_before, ("policy.vanilla.ip_pol_b", [2], b.astype(np.float64), "exact"))
    fx.expected.insert(n_before, ("policy.vanilla.ip_pol_w", [4], w.astype(np.float64), "exact"))
    value(fx)
    fixtures.append((fx, format_dict(network=7, policy=3, value=2, default_activation=1,
                                     input_embedding=2), 2, 0))

    # SE_WITH_HEADFORMAT carrying encoders and smolgen_w: an attention body
    # with RELU_2 FFN and SWISH smolgen, PE_MAP (loader.cpp:110-134); heads
    # from the legacy top-level fields (weights.cpp:245-289).
    fx = Fixture("legacy_se_attention", legacy=True)
    fx.fmt(network=4, policy=3, value=2)
    fx.net.weights.headcount = 2
    body(fx, encoder_layers=1, smolgen=True)
    policy(fx, encoder_layers=1, conv=True)
    fx.net.weights.pol_headcount = 3
    value(fx, conv=True)
    fixtures.append((fx, format_dict(network=6, policy=3, value=2, ffn_activation=8,
                                     smolgen_activation=7, input_embedding=1), 2, 3))

    # No network_format at all: classical 112-plane input, classical heads
    # (loader.cpp:92-100).
    fx = Fixture("no_format", legacy=True)
    policy(fx, conv=True)
    value(fx, conv=True)
    fixtures.append((fx, format_dict(input=1, output=1, network=3, policy=1, value=1,
                                     input_embedding=1), 0, 0))

    # AB_LEGACY_WITH_MULTIHEADFORMAT -> ATTENTIONBODY_WITH_MULTIHEADFORMAT
    # (loader.cpp:117-119); the given input embedding is kept.
    fx = Fixture("ab_legacy")
    fx.fmt(network=134, policy=3, value=2, input_embedding=2, default_activation=1)
    fx.net.weights.headcount = 2
    body(fx, encoder_layers=1, smolgen=False)
    policy(fx)
    value(fx)
    fixtures.append((fx, format_dict(network=7, policy=3, value=2, input_embedding=2,
                                     default_activation=1), 2, 0))

    # NETWORK_CLASSICAL / NETWORK_SE gain the head formats (loader.cpp:102-109).
    for name, net_in, net_out in (("classical", 1, 3), ("se", 2, 4)):
        fx = Fixture(name, legacy=True)
        fx.fmt(input=1, network=net_in, policy=3, value=2, moves_left=0)
        fx.conv("body.input")
        policy(fx, conv=True)
        value(fx)
        fixtures.append((fx, format_dict(input=1, network=net_out, policy=1, value=1,
                                         input_embedding=1), 0, 0))
    return fixtures


def error_fixtures(every_field_bytes):
    out = {}
    n = Net()
    n.magic = 0x1C1
    n.weights.policy_heads.vanilla.ip_pol_w.params = b"\0\0\x80?"
    out["bad_magic"] = (n.SerializeToString(), "Invalid weight file: bad magic number")
    n = Net()
    n.weights.headcount = 1
    out["no_magic"] = (n.SerializeToString(), "Invalid weight file: bad magic number")
    out["truncated"] = (every_field_bytes[:-7], "Failed to parse protobuf weights file")
    out["tiny"] = (b"\x0d", "Invalid weight file: too small")
    n = Net()
    n.magic = 0x1C0
    n.format.network_format.network = 7
    n.weights.encoder.add().mha.rpe_q.params = b"\0\0\0\0"
    n.weights.policy_heads.vanilla.ip_pol_w.params = b"\0\0\x80?"
    n.weights.value_heads.winner.ip_val_w.params = b"\0\0\x80?"
    out["rpe"] = (n.SerializeToString(), "RPE weights file not supported.")
    n = Net()
    n.magic = 0x1C0
    n.weights.ip_emb_w.params = b"\0\0\x80?"
    out["no_policy"] = (n.SerializeToString(), "Could not find valid policy head weights.")
    n = Net()
    n.magic = 0x1C0
    n.weights.ip_pol_w.params = b"\0\0\x80?"
    out["no_value"] = (n.SerializeToString(), "Could not find valid value head weights.")
    return out


def writer_fixtures():
    """Nets for pinning tests/netfile.py: its output for the recorded source
    tensors must equal these libprotobuf-made bytes."""
    out = []
    for name, legacy in (("writer_multihead", False), ("writer_legacy", True)):
        net = Net()
        net.magic = 0x1C0
        fmt = dict(network=7 if not legacy else 6, policy=3, value=2, input_embedding=2,
                   default_activation=1, smolgen_activation=7, ffn_activation=0)
        for k, v in fmt.items():
            setattr(net.format.network_format, k, v)
        net.weights.headcount = 2
        names = ["body." + n for n in BODY_EMBED]
        names += ["body.ip_emb_ffn." + t for t in ("dense1_w", "dense1_b", "dense2_w", "dense2_b")]
        names += ["body.ip_emb_ffn_ln_gammas", "body.ip_emb_ffn_ln_betas", "body.smolgen_w"]
        enc = "body.encoder.0."
        names += [enc + "mha." + t for t in ("q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "dense_w",
                                             "dense_b")]
        names += [enc + "mha.smolgen." + t for t in ("compress", "dense1_w", "dense1_b",
                                                     "ln1_gammas", "ln1_betas", "dense2_w",
                                                     "dense2_b", "ln2_gammas", "ln2_betas")]
        names += [enc + t for t in ("ln1_gammas", "ln1_betas", "ffn.dense1_w", "ffn.dense1_b",
                                    "ffn.dense2_w", "ffn.dense2_b", "ln2_gammas", "ln2_betas")]
        names += ["body.encoder.1.mha.q_w"]
        names += ["policy.vanilla." + n for n in ("ip_pol_w", "ip_pol_b", "ip2_pol_w", "ip2_pol_b",
                                                   "ip3_pol_w", "ip3_pol_b", "ip4_pol_w")]
        names += ["policy.vanilla.encoder.0.mha.k_w", "policy.vanilla.encoder.0.ln1_gammas",
                  "policy.vanilla.policy1.weights", "policy.vanilla.policy.bn_means"]
        names += ["value.winner." + n for n in ("ip_val_w", "ip_val_b", "ip1_val_w", "ip1_val_b",
                                                 "ip2_val_w", "ip2_val_b")]
        names += ["value.winner.value.weights", "value.winner.value.bn_stddivs"]
        if not legacy:
            names += ["value.winner.ip_val_err_w", "value.winner.ip_val_err_b"]
        names += ["moves_left.weights", "moves_left.bn_gammas", "moves_left.ip_mov_w",
                  "moves_left.ip1_mov_b", "moves_left.ip2_mov_w"]
        tensors = []
        for i, n in enumerate(names):
            e = ALL_ENC[i % 5]
            size = 2 + i % 5
            dims = [size] if i % 3 else [1, size]
            v = values_for("f32" if e in ("linear16", "unset") else e, size)
            set_layer(resolve(net, attr_path(n, legacy)), v, e, dims)
            tensors.append((n, v, e, dims))
        if legacy:
            net.weights.pol_headcount = 3
        else:
            net.weights.policy_heads.vanilla.pol_headcount = 3
        out.append((name, legacy, fmt, net.SerializeToString(), tensors))
    return out


def main():
    os.makedirs(OUT, exist_ok=True)
    expected = {}
    arrays = {}
    writer = {}
    for name, legacy, fmt, data, tensors in writer_fixtures():
        with open(os.path.join(OUT, name + ".pb"), "wb") as f:
            f.write(data)
        writer[name] = {"legacy": legacy, "format": fmt, "headcount": 2, "pol_headcount": 3,
                        "tensors": [[n, e, d] for n, _, e, d in tensors]}
        for n, v, _, _ in tensors:
            arrays[f"{name}/{n}"] = v
    every_field = None
    for fx, fmt, heads, pol_heads in build():
        data = fx.net.SerializeToString()
        if fx.name == "every_field":
            every_field = data
        with open(os.path.join(OUT, fx.name + ".pb"), "wb") as f:
            f.write(data)
        expected[fx.name] = {
            "format": fmt, "headcount": heads, "pol_headcount": pol_heads,
            "tensors": [[n, d, kind] for n, d, _, kind in fx.expected]}
        for n, _, v, _ in fx.expected:
            arrays[f"{fx.name}/{n}"] = np.asarray(v, dtype=np.float64)
    # The same bytes gzip-compressed (LoadWeightsFromFile, loader.cpp:165-166).
    with gzip.GzipFile(os.path.join(OUT, "every_field.pb.gz"), "wb", mtime=0) as f:
        f.write(every_field)
    for name, (data, msg) in error_fixtures(every_field).items():
        with open(os.path.join(OUT, name + ".pb"), "wb") as f:
            f.write(data)
        expected[name] = {"error": msg}
    with open(os.path.join(OUT, "expected.json"), "w") as f:
        json.dump({"fixtures": expected, "writer": writer}, f, indent=1, sort_keys=True)
        f.write("\n")
    np.savez_compressed(os.path.join(OUT, "expected.npz"), **arrays)
    print(f"wrote {len(expected) + len(writer)} fixtures to {OUT}", file=sys.stderr)


if __name__ == "__main__":
    main()
