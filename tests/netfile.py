"""Test-side writer of network files in the reference's format
(reference src/nn/proto/net.proto): proto2 wire encoding of a ``Net`` message
from inventory-named tensors, with the Layer encodings the reference's loader
decodes (src/nn/loader.cpp:187-251).

Fields are written in field-number order and repeated ``dims`` unpacked, the
canonical serialisation libprotobuf produces, so the output can be compared
byte for byte with files made by libprotobuf itself (tests/golden/netfiles).
"""

from __future__ import annotations

import gzip
import struct

import numpy as np

ENCODING = {"unset": None, "linear16": 1, "f16": 2, "bf16": 3, "f32": 4}

# Weights (net.proto:169-241), body fields by inventory suffix.
_BODY = {"ip_emb_preproc_w": 37, "ip_emb_preproc_b": 38, "ip_emb_w": 25, "ip_emb_b": 26,
         "ip_emb_ln_gammas": 39, "ip_emb_ln_betas": 40, "ip_mult_gate": 33, "ip_add_gate": 34,
         "ip_emb_ffn_ln_gammas": 42, "ip_emb_ffn_ln_betas": 43, "smolgen_w": 35}
_FFN = {"dense1_w": 1, "dense1_b": 2, "dense2_w": 3, "dense2_b": 4}
_MHA = {"q_w": 1, "q_b": 2, "k_w": 3, "k_b": 4, "v_w": 5, "v_b": 6, "dense_w": 7, "dense_b": 8}
_SMOLGEN = {"compress": 1, "dense1_w": 2, "dense1_b": 3, "ln1_gammas": 4, "ln1_betas": 5,
            "dense2_w": 6, "dense2_b": 7, "ln2_gammas": 8, "ln2_betas": 9}
_ENCODER = {"ln1_gammas": 2, "ln1_betas": 3, "ln2_gammas": 5, "ln2_betas": 6}
_CONV = {"weights": 1, "biases": 2, "bn_means": 3, "bn_stddivs": 4, "bn_gammas": 5,
         "bn_betas": 6}
_POLICY_HEAD = {"ip_pol_w": 1, "ip_pol_b": 2, "ip2_pol_w": 3, "ip2_pol_b": 4, "ip3_pol_w": 5,
                "ip3_pol_b": 6, "ip4_pol_w": 7}
_VALUE_HEAD = {"ip_val_w": 1, "ip_val_b": 2, "ip1_val_w": 3, "ip1_val_b": 4, "ip2_val_w": 5,
               "ip2_val_b": 6, "ip_val_err_w": 7, "ip_val_err_b": 8}
# Top-level legacy head fields (net.proto:201-225).
_LEGACY_POLICY = {"ip_pol_w": 4, "ip_pol_b": 5, "ip2_pol_w": 17, "ip2_pol_b": 18,
                  "ip3_pol_w": 19, "ip3_pol_b": 20, "ip4_pol_w": 22}
_LEGACY_VALUE = {"ip_val_w": 29, "ip_val_b": 30, "ip1_val_w": 7, "ip1_val_b": 8,
                 "ip2_val_w": 9, "ip2_val_b": 10}
_FORMAT = ("input", "output", "network", "policy", "value", "moves_left", "default_activation",
           "smolgen_activation", "ffn_activation", "input_embedding")


def _varint(n: int) -> bytes:
    n &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = n & 0x7F
        n >>= 7
        if n:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(field, wire):
    return _varint((field << 3) | wire)


def f_varint(field, v):
    return _key(field, 0) + _varint(v)


def f_fixed32(field, v):
    return _key(field, 5) + struct.pack("<I", v)


def f_float(field, v):
    return _key(field, 5) + struct.pack("<f", v)


def f_bytes(field, b):
    return _key(field, 2) + _varint(len(b)) + bytes(b)


def bf16_round(x):
    """fp32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def linear16_codes(x):
    """LINEAR16 codes of x over [min, max] (nearest code)."""
    x = np.asarray(x, dtype=np.float64)
    lo, hi = float(np.float32(x.min())), float(np.float32(x.max()))
    if hi == lo:
        return np.zeros(x.shape, np.uint16), lo, hi
    q = np.rint((x - lo) / (hi - lo) * 65535.0)
    return np.clip(q, 0, 65535).astype(np.uint16), lo, hi


def layer(values, encoding="f32", dims=None) -> bytes:
    """A serialised Weights.Layer (net.proto:18-31)."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = b""
    if encoding in ("linear16", "unset"):
        q, lo, hi = linear16_codes(v)
        out += f_float(1, lo) + f_float(2, hi)
        params = q.astype("<u2").tobytes()
    elif encoding == "f16":
        params = v.astype("<f2").tobytes()
    elif encoding == "bf16":
        params = bf16_round(v).astype("<u2").tobytes()
    elif encoding == "f32":
        params = v.astype("<f4").tobytes()
    else:
        raise ValueError(encoding)
    out += f_bytes(3, params)
    if ENCODING[encoding] is not None:
        out += f_varint(4, ENCODING[encoding])
    for d in (dims if dims is not None else [v.size]):
        out += f_varint(5, int(d))
    return out


def _serialise(node) -> bytes:
    """node: {field: bytes | int | node | [node | bytes, ...]} in any order."""
    out = []
    for field in sorted(node):
        val = node[field]
        items = val if isinstance(val, list) else [val]
        for item in items:
            if isinstance(item, dict):
                out.append(f_bytes(field, _serialise(item)))
            elif isinstance(item, (bytes, bytearray)):
                out.append(f_bytes(field, item))
            else:
                out.append(f_varint(field, int(item)))
    return b"".join(out)


def _child(node, field, index=None):
    if index is None:
        return node.setdefault(field, {})
    lst = node.setdefault(field, [])
    while len(lst) <= index:
        lst.append({})
    return lst[index]


def _place_encoder(node, rest, blob):
    if rest[0] == "mha":
        mha = _child(node, 1)
        if rest[1] == "smolgen":
            _child(mha, 9)[_SMOLGEN[rest[2]]] = blob
        else:
            mha[_MHA[rest[1]]] = blob
    elif rest[0] == "ffn":
        _child(node, 4)[_FFN[rest[1]]] = blob
    else:
        node[_ENCODER[rest[0]]] = blob


def _place(weights, name, blob, legacy_heads):
    parts = name.split(".")
    if parts[0] == "body":
        if parts[1] == "encoder":
            _place_encoder(_child(weights, 27, int(parts[2])), parts[3:], blob)
        elif parts[1] == "ip_emb_ffn":
            _child(weights, 41)[_FFN[parts[2]]] = blob
        elif parts[1] == "input":
            _child(weights, 1)[_CONV[parts[2]]] = blob
        elif parts[1] == "residual":
            res = _child(weights, 2, int(parts[2]))
            if parts[3] == "se":
                _child(res, 3)[{"w1": 1, "b1": 2, "w2": 3, "b2": 4}[parts[4]]] = blob
            else:
                _child(res, {"conv1": 1, "conv2": 2}[parts[3]])[_CONV[parts[4]]] = blob
        else:
            weights[_BODY[parts[1]]] = blob
    elif parts[0] == "policy":
        rest = parts[2:]
        if legacy_heads:
            if rest[0] == "encoder":
                _place_encoder(_child(weights, 21, int(rest[1])), rest[2:], blob)
            elif rest[0] in ("policy1", "policy"):
                _child(weights, {"policy1": 11, "policy": 3}[rest[0]])[_CONV[rest[1]]] = blob
            else:
                weights[_LEGACY_POLICY[rest[0]]] = blob
        else:
            head = _child(_child(weights, 45), 3)
            if rest[0] == "encoder":
                _place_encoder(_child(head, 8, int(rest[1])), rest[2:], blob)
            elif rest[0] in ("policy1", "policy"):
                _child(head, {"policy1": 10, "policy": 11}[rest[0]])[_CONV[rest[1]]] = blob
            else:
                head[_POLICY_HEAD[rest[0]]] = blob
    elif parts[0] == "value":
        rest = parts[2:]
        if legacy_heads:
            if rest[0] == "value":
                _child(weights, 6)[_CONV[rest[1]]] = blob
            else:
                weights[_LEGACY_VALUE[rest[0]]] = blob
        else:
            head = _child(_child(weights, 44), 1)
            if rest[0] == "value":
                _child(head, 11)[_CONV[rest[1]]] = blob
            else:
                head[_VALUE_HEAD[rest[0]]] = blob
    elif parts[0] == "moves_left":
        if parts[1] in _CONV:
            _child(weights, 12)[_CONV[parts[1]]] = blob
        else:
            weights[{"ip_mov_w": 31, "ip_mov_b": 32, "ip1_mov_w": 13, "ip1_mov_b": 14,
                     "ip2_mov_w": 15, "ip2_mov_b": 16}[parts[1]]] = blob
    else:
        raise KeyError(name)


def net_bytes(tensors, fmt=None, headcount=None, pol_headcount=None, encoding="f32",
              legacy_heads=False, magic=0x1C0, dims=None) -> bytes:
    """Serialised Net (net.proto:371-379).  ``tensors``: {inventory name:
    array}; ``fmt``: NetworkFormat fields by name (None: no network_format);
    ``encoding``: one Layer encoding for all tensors or {name: encoding};
    ``dims``: optional {name: dims list}."""
    weights = {}
    for name, arr in tensors.items():
        enc = encoding if isinstance(encoding, str) else encoding.get(name, "f32")
        d = None if dims is None else dims.get(name)
        _place(weights, name, layer(arr, enc, d), legacy_heads)
    if headcount is not None:
        weights[28] = int(headcount)
    if pol_headcount is not None:
        if legacy_heads:
            weights[24] = int(pol_headcount)
        else:
            _child(_child(weights, 45), 3)[9] = int(pol_headcount)
    net = {}
    out = f_fixed32(1, magic) if magic is not None else b""
    if fmt is not None:
        # NetworkFormat fields 1..10 in _FORMAT order (net.proto:253-343).
        net[4] = {2: {i + 1: int(fmt[k]) for i, k in enumerate(_FORMAT) if k in fmt}}
    if weights:
        net[10] = weights
    return out + _serialise(net)


def decoded(values, encoding):
    """fp32 values the loader yields for ``values`` written with ``encoding``
    (exact for f32/f16/bf16; LINEAR16 by its definition, in float32)."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    if encoding == "f32":
        return v.copy()
    if encoding == "f16":
        return v.astype(np.float16).astype(np.float32)
    if encoding == "bf16":
        return (bf16_round(v).astype(np.uint32) << 16).view(np.float32)
    q, lo, hi = linear16_codes(v)
    lo32, hi32 = np.float32(lo), np.float32(hi)
    return (lo32 + (q.astype(np.float32) / np.float32(65535.0)) * (hi32 - lo32)).astype(np.float32)


def write(path, data: bytes):
    if str(path).endswith(".gz"):
        with gzip.open(path, "wb") as f:
            f.write(data)
    else:
        with open(path, "wb") as f:
            f.write(data)


_ACTIVATION = {"default": 0, "mish": 1, "relu": 2, "none": 3, "tanh": 4, "sigmoid": 5,
               "selu": 6, "swish": 7, "relu_2": 8}


def spec_net_bytes(spec, weights, layout):
    """A synth.NetSpec net as a multi-head attention-body file (PE_DENSE);
    ``layout`` is synth.tensor_layout(spec).  GEMM matrices go out as
    BFLOAT16 (they hold bf16 values, so exactly), the rest as FLOAT32."""
    enc = {name: ("bf16" if bf16 else "f32") for name, _, _, _, bf16 in layout}
    fmt = dict(network=7, policy=3, value=2 if spec.wdl else 1, input_embedding=2,
               default_activation=1 if spec.default_activation == "mish" else 0,
               ffn_activation=_ACTIVATION[spec.ffn_activation],
               smolgen_activation=_ACTIVATION[spec.smolgen_activation])
    return net_bytes(weights, fmt, spec.heads, encoding=enc)
