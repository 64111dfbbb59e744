"""Seeded synthetic nets and positions (ctypes over libmfhost.so).

Net shapes are the benchmark configurations: ``cpu_plumbing`` (2 layers,
d_model 256) and ``bt4`` (15 layers, d_model 1024, 32 heads, FFN 1536,
smolgen 32 -> 256 -> 32 x 256).  Tensor names are the reference's weight
inventory names and matrices are [out][in].  Builder choices the reference
leaves open: dynamic PE width 16 (concat 112+16 = 128), input-embedding
LayerNorm + gates + FFN present, policy width = d_model, value widths 32/128,
weights N(0, 1/fan_in) (biases too), LayerNorm gamma / mult gate
1 + 0.1 N(0,1), beta / add gate 0.1 N(0,1).  Matrices the GPU multiplies on
MFMA are stored rounded to bf16 values so that the CPU oracle and the GPU
see identical weights.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
_lib = None

NORMAL, ONE_PLUS_TENTH, TENTH, ZERO = 0, 1, 2, 3


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(_PKG, "libmfhost.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run __graft_entry__.build()")
        _lib = ctypes.CDLL(path)
        _lib.mfs_fill_tensor.argtypes = [ctypes.c_uint64, ctypes.c_char_p, ctypes.c_int,
                                         ctypes.c_double, ctypes.c_void_p, ctypes.c_uint64]
        _lib.mfs_round_bf16.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        _lib.mfs_playout_batch.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        _lib.mfs_encode_game.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_int]
        _lib.mfs_encode_game_format.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int,
                                                ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                                ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        _lib.mfs_move_to_index.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_char,
                                           ctypes.c_int]
        _lib.mfs_index_to_move.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_void_p]
        _lib.mfs_perft.argtypes = [ctypes.c_char_p, ctypes.c_int]
        _lib.mfs_perft.restype = ctypes.c_int64
        _lib.mfs_policy_tables.argtypes = [ctypes.c_void_p] * 3
        _lib.mfs_static_position_encoding.argtypes = [ctypes.c_void_p]
    return _lib


@dataclass(frozen=True)
class NetSpec:
    name: str
    embedding: int
    layers: int
    heads: int
    ffn: int
    pe_channels: int = 16
    input_ffn: int = 0
    smolgen_compress: int = 0
    smolgen_hidden: int = 0
    smolgen_gen: int = 0
    policy_dim: int = 0
    value_dim: int = 32
    value_hidden: int = 128
    pe_map: bool = False         # static position encoding (PE_MAP) instead of PE_DENSE
    policy_encoders: int = 0     # encoder layers in the policy head
    policy_heads: int = 0        # their attention heads
    moves_left_dim: int = 0      # moves-left head square embedding (0: no head)
    moves_left_hidden: int = 128
    wdl: bool = True
    gates: bool = True
    default_activation: str = "mish"
    ffn_activation: str = "mish"
    smolgen_activation: str = "swish"


SPECS = {
    # CPU-runnable plumbing net.
    "cpu_plumbing": NetSpec("cpu_plumbing", 256, 2, 8, 512, input_ffn=512, policy_dim=256),
    # BT4-shape net.
    "bt4": NetSpec("bt4", 1024, 15, 32, 1536, input_ffn=1536, smolgen_compress=32,
                   smolgen_hidden=256, smolgen_gen=256, policy_dim=1024),
    # Test net: config 1 plus a moves-left head (8-channel square embedding,
    # 128 hidden, the Lc0 widths).
    "cpu_plumbing_mlh": NetSpec("cpu_plumbing_mlh", 256, 2, 8, 512, input_ffn=512,
                                policy_dim=256, moves_left_dim=8),
    # Test net: config 1 with the PE_MAP static position encoding (64
    # channels, embedding input 112 + 64) in place of the dynamic one.
    "cpu_plumbing_pe_map": NetSpec("cpu_plumbing_pe_map", 256, 2, 8, 512, pe_channels=64,
                                   input_ffn=512, policy_dim=256, pe_map=True),
    # Test net: config 1 with smolgen (16 compressed channels -> 64 hidden ->
    # 8 heads x 64 gen): 8 heads per position, so the attention kernel's
    # groups of 16 (position, head) pairs span two positions.
    "cpu_plumbing_smolgen": NetSpec("cpu_plumbing_smolgen", 256, 2, 8, 512, input_ffn=512,
                                    smolgen_compress=16, smolgen_hidden=64, smolgen_gen=64,
                                    policy_dim=256),
    # Test net: config 1 with one encoder layer (8 heads) in the policy head.
    "cpu_plumbing_pol_enc": NetSpec("cpu_plumbing_pol_enc", 256, 2, 8, 512, input_ffn=512,
                                    policy_dim=256, policy_encoders=1, policy_heads=8),
}


def tensor_layout(spec: NetSpec):
    """(name, shape, init kind, fan_in, stored as bf16) for every tensor."""
    E, P, S = spec.embedding, spec.pe_channels, 64
    out = []

    def mat(name, rows, cols, bf16=True):
        out.append((name, (rows, cols), NORMAL, cols, bf16))

    def vec(name, n, fan_in, kind=NORMAL):
        out.append((name, (n,), kind, fan_in, False))

    def norm(prefix, n):
        vec(prefix + "_gammas", n, 0, ONE_PLUS_TENTH)
        vec(prefix + "_betas", n, 0, TENTH)

    if not spec.pe_map:
        mat("body.ip_emb_preproc_w", S * P, S * 12)
        vec("body.ip_emb_preproc_b", S * P, S * 12)
    mat("body.ip_emb_w", E, 112 + P)
    vec("body.ip_emb_b", E, 112 + P)
    norm("body.ip_emb_ln", E)
    if spec.gates:
        vec("body.ip_mult_gate", E * S, 0, ONE_PLUS_TENTH)
        vec("body.ip_add_gate", E * S, 0, TENTH)
    if spec.input_ffn:
        mat("body.ip_emb_ffn.dense1_w", spec.input_ffn, E)
        vec("body.ip_emb_ffn.dense1_b", spec.input_ffn, E)
        mat("body.ip_emb_ffn.dense2_w", E, spec.input_ffn)
        vec("body.ip_emb_ffn.dense2_b", E, spec.input_ffn)
        norm("body.ip_emb_ffn_ln", E)
    if spec.smolgen_compress:
        mat("body.smolgen_w", S * S, spec.smolgen_gen)
    for i in range(spec.layers):
        p = f"body.encoder.{i}"
        for t in ("q", "k", "v"):
            mat(f"{p}.mha.{t}_w", E, E)
            vec(f"{p}.mha.{t}_b", E, E)
        mat(f"{p}.mha.dense_w", E, E)
        vec(f"{p}.mha.dense_b", E, E)
        if spec.smolgen_compress:
            c, h, g = spec.smolgen_compress, spec.smolgen_hidden, spec.smolgen_gen
            sg = f"{p}.mha.smolgen"
            mat(sg + ".compress", c, E)
            mat(sg + ".dense1_w", h, S * c)
            vec(sg + ".dense1_b", h, S * c)
            mat(sg + ".dense2_w", spec.heads * g, h)
            vec(sg + ".dense2_b", spec.heads * g, h)
            norm(sg + ".ln1", h)
            norm(sg + ".ln2", spec.heads * g)
        norm(f"{p}.ln1", E)
        mat(f"{p}.ffn.dense1_w", spec.ffn, E)
        vec(f"{p}.ffn.dense1_b", spec.ffn, E)
        mat(f"{p}.ffn.dense2_w", E, spec.ffn)
        vec(f"{p}.ffn.dense2_b", E, spec.ffn)
        norm(f"{p}.ln2", E)
    for i in range(spec.policy_encoders):
        p = f"policy.vanilla.encoder.{i}"
        for t in ("q", "k", "v"):
            mat(f"{p}.mha.{t}_w", E, E)
            vec(f"{p}.mha.{t}_b", E, E)
        mat(f"{p}.mha.dense_w", E, E)
        vec(f"{p}.mha.dense_b", E, E)
        norm(f"{p}.ln1", E)
        mat(f"{p}.ffn.dense1_w", spec.ffn, E)
        vec(f"{p}.ffn.dense1_b", spec.ffn, E)
        mat(f"{p}.ffn.dense2_w", E, spec.ffn)
        vec(f"{p}.ffn.dense2_b", E, spec.ffn)
        norm(f"{p}.ln2", E)
    dp = spec.policy_dim
    mat("policy.vanilla.ip_pol_w", dp, E)
    vec("policy.vanilla.ip_pol_b", dp, E)
    mat("policy.vanilla.ip2_pol_w", dp, dp)
    vec("policy.vanilla.ip2_pol_b", dp, dp)
    mat("policy.vanilla.ip3_pol_w", dp, dp)
    vec("policy.vanilla.ip3_pol_b", dp, dp)
    mat("policy.vanilla.ip4_pol_w", 4, dp, bf16=False)
    vd, vh = spec.value_dim, spec.value_hidden
    mat("value.winner.ip_val_w", vd, E)
    vec("value.winner.ip_val_b", vd, E)
    mat("value.winner.ip1_val_w", vh, S * vd)
    vec("value.winner.ip1_val_b", vh, S * vd)
    nout = 3 if spec.wdl else 1
    mat("value.winner.ip2_val_w", nout, vh, bf16=False)
    vec("value.winner.ip2_val_b", nout, vh)
    if spec.moves_left_dim:
        md, mh = spec.moves_left_dim, spec.moves_left_hidden
        mat("moves_left.ip_mov_w", md, E)
        vec("moves_left.ip_mov_b", md, E)
        mat("moves_left.ip1_mov_w", mh, S * md)
        vec("moves_left.ip1_mov_b", mh, S * md)
        mat("moves_left.ip2_mov_w", 1, mh, bf16=False)
        vec("moves_left.ip2_mov_b", 1, mh)
    return out


def e4m3_encode(x):
    """OCP e4m3 codes of float32 ``x`` (round to nearest even, saturating at
    +-448), the encoding the fp8 weight storage uses."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    au = u & 0x7FFFFFFF
    a = au.astype(np.uint32).view(np.float32)
    sub = a < np.float32(0.015625)
    code_sub = np.rint(a * np.float32(512.0)).astype(np.int64)
    r = au + 0x7FFFF + ((au >> 20) & 1)
    e = (r >> 23).astype(np.int64) - 127
    m = ((r >> 20) & 7).astype(np.int64)
    code_n = np.where((e > 8) | ((e == 8) & (m == 7)), 0x7E, ((e + 7) << 3) | m)
    return (sign | np.where(sub, code_sub, code_n).astype(np.uint8)).astype(np.uint8)


def e4m3_values():
    """float32 value of each of the 256 e4m3 codes (NaN for 0x7F / 0xFF)."""
    v = np.empty(256, np.float32)
    for c in range(256):
        e, m = (c >> 3) & 15, c & 7
        mag = (1 + m / 8.0) * 2.0 ** (e - 7) if e else m * 2.0 ** -9
        v[c] = np.nan if (c & 0x7F) == 0x7F else (-mag if c & 0x80 else mag)
    return v


def quantize_fp8_rows(w):
    """Per-row e4m3 quantisation of a [rows, cols] matrix: (codes, scales,
    dequantised fp32 values), scale = max|row| / 448."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(w.shape[0], -1)
    mx = np.abs(w).max(axis=1)
    scale = np.where(mx > 0, mx / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    codes = e4m3_encode(w / scale[:, None])
    deq = (e4m3_values()[codes] * scale[:, None]).astype(np.float32)
    return codes, scale, deq


def make_weights(spec: NetSpec, seed: int = 0, quantize: bool = True, fp8: bool = False):
    """Deterministic fp32 weights {name: ndarray}; GEMM matrices rounded to
    bf16-representable values when ``quantize``, or to their per-row e4m3
    dequantised values when ``fp8`` (the values an fp8-weight net computes
    with)."""
    L = lib()
    weights = {}
    for name, shape, kind, fan_in, bf16 in tensor_layout(spec):
        arr = np.empty(shape, dtype=np.float32)
        L.mfs_fill_tensor(seed, name.encode(), kind, float(fan_in), arr.ctypes.data, arr.size)
        if bf16 and fp8:
            arr = quantize_fp8_rows(arr.reshape(shape[0], -1))[2].reshape(shape)
        elif bf16 and quantize:
            L.mfs_round_bf16(arr.ctypes.data, arr.size)
        weights[name] = arr
    return weights


def parameter_count(spec: NetSpec) -> int:
    return sum(int(np.prod(s)) for _, s, _, _, _ in tensor_layout(spec))


def playout_positions(count: int, seed: int = 0, first_game: int = 0, min_plies: int = 10,
                      max_plies: int = 60, with_moves: bool = False):
    """Seeded random-playout positions encoded as planes [count,112,64],
    plus legal-move policy indices [count,256] (-1 padded)."""
    planes = np.zeros((count, 112, 64), dtype=np.float32)
    legal = np.full((count, 256), -1, dtype=np.int16)
    stride = 1024
    text = ctypes.create_string_buffer(count * stride) if with_moves else None
    rc = lib().mfs_playout_batch(seed, first_game, count, min_plies, max_plies,
                                 planes.ctypes.data, legal.ctypes.data, text,
                                 stride if with_moves else 0)
    if rc != 0:
        raise RuntimeError(f"playout generation failed ({rc})")
    if with_moves:
        moves = [text.raw[i * stride:(i + 1) * stride].split(b"\0", 1)[0].decode()
                 for i in range(count)]
        return planes, legal, moves
    return planes, legal


def encode_game(fen: str = "", moves: str = ""):
    planes = np.zeros((112, 64), dtype=np.float32)
    legal = np.full((256,), -1, dtype=np.int16)
    n = lib().mfs_encode_game(fen.encode(), moves.encode(), planes.ctypes.data,
                              legal.ctypes.data, 256)
    if n < 0:
        raise ValueError(f"cannot encode game fen={fen!r} moves={moves!r}")
    return planes, legal[:n]


# net.proto InputFormat values.
INPUT_FORMATS = {"classical": 1, "castling_plane": 2, "canonical": 3,
                 "canonical_hectoplies": 4, "canonical_hectoplies_armageddon": 132,
                 "canonical_v2": 5, "canonical_v2_armageddon": 133}
FILL = {"no": 0, "fen_only": 1, "always": 2}


def encode_game_format(fen: str = "", moves: str = "", input_format="classical",
                       fill="fen_only", history_planes=8):
    """EncodePositionForNN for any input format: (planes [112, 64], legal
    policy indices under the chosen transform, transform)."""
    planes = np.zeros((112, 64), dtype=np.float32)
    legal = np.full((256,), -1, dtype=np.int16)
    t = ctypes.c_int(0)
    fmt = INPUT_FORMATS.get(input_format, input_format)
    n = lib().mfs_encode_game_format(fen.encode(), moves.encode(), int(fmt), FILL[fill],
                                     history_planes, planes.ctypes.data, legal.ctypes.data,
                                     256, ctypes.byref(t))
    if n < 0:
        raise ValueError(f"cannot encode game fen={fen!r} moves={moves!r} format={fmt}")
    return planes, legal[:n], t.value


def move_to_index(frm: int, to: int, promo: str = "", transform: int = 0) -> int:
    return lib().mfs_move_to_index(frm, to, promo.encode() if promo else b"\0", transform)


def index_to_move(index: int, transform: int = 0):
    f, t, p = ctypes.c_int(), ctypes.c_int(), ctypes.c_char()
    if lib().mfs_index_to_move(index, transform, ctypes.byref(f), ctypes.byref(t),
                               ctypes.byref(p)) != 0:
        raise ValueError(f"bad policy index {index}")
    return f.value, t.value, p.value.decode() if p.value != b"\0" else ""


def perft(fen: str, depth: int) -> int:
    n = lib().mfs_perft(fen.encode(), depth)
    if n < 0:
        raise ValueError("invalid FEN")
    return int(n)


def policy_tables():
    amap = np.zeros(4288, dtype=np.int16)
    gather = np.zeros(1858, dtype=np.int16)
    strings = ctypes.create_string_buffer(1858 * 6)
    lib().mfs_policy_tables(amap.ctypes.data, gather.ctypes.data, strings)
    names = [strings.raw[6 * i:6 * i + 6].split(b"\0", 1)[0].decode() for i in range(1858)]
    return amap, gather, names


def static_position_encoding():
    """The PE_MAP static position encoding [64 squares, 64 channels]."""
    out = np.zeros((64, 64), dtype=np.float32)
    lib().mfs_static_position_encoding(out.ctypes.data)
    return out
