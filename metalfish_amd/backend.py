"""Python binding of the C ABI in include/mfhip.h (libmfhip.so).

``HipNetwork`` mirrors the reference's ``NN::Network`` operations
(reference src/nn/network.h:38-51): ``evaluate`` / ``evaluate_batch`` return
raw 1858 policy logits, WDL and value = W - L
(reference src/nn/network_output_decoder.cpp:56-63); ``info()`` and
``capabilities()`` stand for GetNetworkInfo / GetBackendCapabilities.
There is no CPU fallback: without the library or a gfx950 device every call
raises.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libmfhip.so")

MFH_OK = 0
PRECISION = {"bf16": 0, "bf16x2": 1, "bf16x2_gemm": 2, "fp8": 3, "bf16x2_fp8lo": 4}
WEIGHTS = {"bf16": 0, "fp8": 1}
ACTIVATION = {"default": 0, "mish": 1, "relu": 2, "none": 3, "tanh": 4, "sigmoid": 5,
              "selu": 6, "swish": 7, "relu_2": 8}

# Every symbol include/mfhip.h declares.
EXPORTS = ("mfh_net_create", "mfh_net_destroy", "mfh_net_eval", "mfh_net_eval_planes",
           "mfh_net_eval_device", "mfh_net_info", "mfh_net_capabilities",
           "mfh_net_set_graphs", "mfh_net_set_profiling", "mfh_net_profile",
           "mfh_net_profile_reset",
           "mfh_pack_planes", "mfh_device_count", "mfh_last_error", "mfh_debug_unpack_planes",
           "mfh_debug_gemm_bf16", "mfh_debug_panel_gemm", "mfh_net_debug_tensor", "mfh_debug_quantize_fp8",
           "mfh_weights_load", "mfh_weights_parse", "mfh_weights_describe",
           "mfh_weights_tensors", "mfh_weights_tensor_dims", "mfh_weights_free",
           "mfh_net_eval_priors", "mfh_net_eval_priors_device",
           "mfh_net_eval_device_moves_left", "mfh_net_eval_device_noalloc",
           "mfh_debug_encoder_layer", "mfh_debug_skinny_gemm", "mfh_debug_gemm_fp8",
           "mfh_debug_quantize_rows_e4m3", "mfh_debug_gemm_lo8")
FORMAT_FIELDS = ("input", "output", "network", "policy", "value", "moves_left",
                 "default_activation", "smolgen_activation", "ffn_activation", "input_embedding")


class MfhNetDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "network", "policy", "value", "moves_left", "input_embedding", "default_activation",
        "ffn_activation", "smolgen_activation", "headcount", "weights_dtype", "precision",
        "max_batch", "device", "pol_headcount", "fused_layernorm")]


class MfhTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("data", ctypes.c_void_p), ("count", ctypes.c_uint64)]


class MfhWeightsFormat(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in FORMAT_FIELDS + ("headcount", "pol_headcount")]


class MfhProfileEntry(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("launches", ctypes.c_int),
                ("milliseconds", ctypes.c_double), ("flops", ctypes.c_double),
                ("bytes", ctypes.c_double)]


class MfhCapabilities(ctypes.Structure):
    _fields_ = [("has_wdl", ctypes.c_int), ("has_moves_left", ctypes.c_int),
                ("max_batch_size", ctypes.c_int), ("device", ctypes.c_int),
                ("device_name", ctypes.c_char * 64), ("arch_name", ctypes.c_char * 32),
                ("weight_bytes", ctypes.c_uint64), ("workspace_bytes", ctypes.c_uint64)]


_lib = None


def lib():
    """Loads libmfhip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP backend library missing: {LIB_PATH} "
                               "(run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        vp, i, u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64
        sig = {
            "mfh_net_create": ([ctypes.POINTER(MfhNetDesc), vp, i, ctypes.POINTER(vp)], i),
            "mfh_net_destroy": ([vp], None),
            "mfh_net_eval": ([vp, i, vp, vp, vp, vp, vp], i),
            "mfh_net_eval_planes": ([vp, i, vp, vp, vp, vp], i),
            "mfh_net_eval_device": ([vp, i, vp, vp, vp, vp, vp], i),
            "mfh_net_info": ([vp, ctypes.c_char_p, ctypes.c_size_t], i),
            "mfh_net_capabilities": ([vp, ctypes.POINTER(MfhCapabilities)], i),
            "mfh_net_set_graphs": ([vp, i], i),
            "mfh_net_set_profiling": ([vp, i], i),
            "mfh_net_profile": ([vp, ctypes.POINTER(MfhProfileEntry), i, ctypes.POINTER(i)], i),
            "mfh_net_profile_reset": ([vp], i),
            "mfh_pack_planes": ([i, vp, vp, vp], i),
            "mfh_device_count": ([ctypes.POINTER(i)], i),
            "mfh_last_error": ([], ctypes.c_char_p),
            "mfh_debug_unpack_planes": ([i, vp, vp, vp], i),
            "mfh_debug_gemm_bf16": ([i, i, i, vp, vp, vp, i, vp], i),
            "mfh_debug_panel_gemm": ([i, i, i, vp, vp, vp, vp, vp, vp, i, i, vp, vp, vp,
                                      ctypes.c_float, ctypes.c_float, vp, vp, vp, vp, vp], i),
            "mfh_debug_skinny_gemm": ([i, i, i, vp, vp, vp, i, ctypes.c_float, vp, vp, i, vp, vp,
                                       i, i, vp, vp, vp, ctypes.c_float, vp, vp, vp,
                                       ctypes.POINTER(i), vp, vp, vp], i),
            "mfh_debug_gemm_fp8": ([i, i, i, vp, vp, vp, vp, vp, i, vp], i),
            "mfh_debug_gemm_lo8": ([i, i, i, vp, vp, vp, vp, vp, vp, i, vp, vp, vp], i),
            "mfh_debug_quantize_rows_e4m3": ([i, i, vp, vp, vp, vp], i),
            "mfh_net_debug_tensor": ([vp, ctypes.c_char_p, vp, u64], i),
            "mfh_debug_quantize_fp8": ([i, i, vp, vp, vp], i),
            "mfh_weights_load": ([ctypes.c_char_p, ctypes.POINTER(vp)], i),
            "mfh_weights_parse": ([vp, u64, ctypes.POINTER(vp)], i),
            "mfh_weights_describe": ([vp, ctypes.POINTER(MfhWeightsFormat),
                                      ctypes.POINTER(MfhNetDesc)], i),
            "mfh_weights_tensors": ([vp, ctypes.POINTER(ctypes.POINTER(MfhTensor)),
                                     ctypes.POINTER(i)], i),
            "mfh_weights_tensor_dims": ([vp, i, ctypes.POINTER(ctypes.POINTER(ctypes.c_uint32)),
                                         ctypes.POINTER(i)], i),
            "mfh_weights_free": ([vp], None),
            "mfh_net_eval_priors": ([vp, i, vp, vp, vp, vp, ctypes.c_float, vp, vp, vp], i),
            "mfh_net_eval_priors_device": ([vp, i, vp, vp, vp, vp, ctypes.c_float, vp, vp, vp,
                                            vp], i),
            "mfh_net_eval_device_moves_left": ([vp, i, vp, vp, vp, vp, vp, vp], i),
            "mfh_net_eval_device_noalloc": ([vp, i, vp, vp, vp, vp, vp], i),
            "mfh_debug_encoder_layer": ([vp, i, i, i, vp, vp, ctypes.POINTER(ctypes.c_float)], i),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _check(rc, what):
    if rc != MFH_OK:
        msg = lib().mfh_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(lib().mfh_device_count(ctypes.byref(n)), "mfh_device_count")
    return n.value


def _ptr(a):
    return a.ctypes.data if a is not None else None


class HipNetwork:
    """Attention-body network resident on one MI355X."""

    def __init__(self, weights: dict, heads: int, *, wdl=True, default_activation="mish",
                 ffn_activation="default", smolgen_activation="swish", max_batch=256,
                 device=-1, precision="bf16x2", weights_dtype="bf16", net_format=None,
                 moves_left=False, pe_map=False, pol_heads=0, fused_layernorm=False):
        """``net_format``: NetworkFormat fields of a loaded file
        (``WeightsFile.format``); they replace the description the keyword
        arguments give.  ``fused_layernorm``: residual GEMM + LayerNorm as one
        row-panel launch at batches >= 128 (split precisions)."""
        self._weights = {k: np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
                         for k, v in weights.items()}
        names = list(self._weights)
        self._names = [n.encode() for n in names]
        tensors = (MfhTensor * len(names))()
        for j, n in enumerate(names):
            a = self._weights[n]
            tensors[j] = MfhTensor(self._names[j], a.ctypes.data, a.size)
        desc = MfhNetDesc(network=6, policy=3, value=2 if wdl else 1,
                          moves_left=1 if moves_left else 0,
                          input_embedding=1 if pe_map else 2,
                          default_activation=1 if default_activation == "mish" else 0,
                          ffn_activation=ACTIVATION[ffn_activation],
                          smolgen_activation=ACTIVATION[smolgen_activation], headcount=heads,
                          weights_dtype=WEIGHTS[weights_dtype], precision=PRECISION[precision],
                          max_batch=max_batch, device=device, pol_headcount=pol_heads,
                          fused_layernorm=1 if fused_layernorm else 0)
        if net_format is not None:
            for k in ("network", "policy", "value", "moves_left", "input_embedding",
                      "default_activation", "ffn_activation", "smolgen_activation"):
                setattr(desc, k, int(net_format[k]))
            wdl = net_format["value"] == 2
            moves_left = net_format["moves_left"] == 1
        handle = ctypes.c_void_p()
        self._h = None
        _check(lib().mfh_net_create(ctypes.byref(desc), tensors, len(names),
                                    ctypes.byref(handle)), "mfh_net_create")
        self._h = handle
        self.wdl = wdl
        self.moves_left = bool(moves_left)
        self.max_batch = max_batch
        self.precision = precision
        self.weights_dtype = weights_dtype
        # Host weights are only needed for the upload.
        self._weights = None

    def close(self):
        if self._h:
            lib().mfh_net_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> str:
        buf = ctypes.create_string_buffer(1024)
        _check(lib().mfh_net_info(self._h, buf, len(buf)), "mfh_net_info")
        return buf.value.decode()

    def capabilities(self) -> dict:
        c = MfhCapabilities()
        _check(lib().mfh_net_capabilities(self._h, ctypes.byref(c)), "mfh_net_capabilities")
        return {"actual_backend": "hip", "has_wdl": bool(c.has_wdl),
                "has_moves_left": bool(c.has_moves_left), "max_batch_size": c.max_batch_size,
                "device": c.device, "device_name": c.device_name.decode(),
                "arch": c.arch_name.decode(), "weight_bytes": c.weight_bytes,
                "workspace_bytes": c.workspace_bytes}

    def _outputs(self, b):
        return (np.zeros((b, 1858), np.float32),
                np.zeros((b, 3 if self.wdl else 1), np.float32))

    def eval_packed(self, masks, values, with_moves_left=False):
        """Raw outputs (policy [B,1858], wdl [B,3] or value [B,1], and with
        ``with_moves_left`` the moves-left output [B]) for packed inputs,
        chunked by max_batch."""
        masks = np.ascontiguousarray(masks, dtype=np.uint64).reshape(-1, 112)
        values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1, 112)
        b = masks.shape[0]
        policy, value = self._outputs(b)
        ml = np.zeros(b, np.float32) if with_moves_left else None
        for s in range(0, b, self.max_batch):
            e = min(b, s + self.max_batch)
            _check(lib().mfh_net_eval(self._h, e - s, _ptr(masks[s:e]), _ptr(values[s:e]),
                                      _ptr(policy[s:e]), _ptr(value[s:e]),
                                      None if ml is None else _ptr(ml[s:e])),
                   "mfh_net_eval")
        return (policy, value, ml) if with_moves_left else (policy, value)

    def eval_planes(self, planes, with_moves_left=False):
        planes = np.ascontiguousarray(planes, dtype=np.float32).reshape(-1, 112, 64)
        b = planes.shape[0]
        policy, value = self._outputs(b)
        ml = np.zeros(b, np.float32) if with_moves_left else None
        for s in range(0, b, self.max_batch):
            e = min(b, s + self.max_batch)
            _check(lib().mfh_net_eval_planes(self._h, e - s, _ptr(planes[s:e]),
                                             _ptr(policy[s:e]), _ptr(value[s:e]),
                                             None if ml is None else _ptr(ml[s:e])),
                   "mfh_net_eval_planes")
        return (policy, value, ml) if with_moves_left else (policy, value)

    def eval_priors(self, masks, values, moves, softmax_temp=1.0):
        """MCTS priors of each position's legal moves, computed on the device
        (mfh_net_eval_priors).  ``moves``: one sequence of policy indices per
        position (at most 256).  Returns (list of float32 prior arrays, raw
        value head output [B, 3] or [B, 1])."""
        masks = np.ascontiguousarray(masks, dtype=np.uint64).reshape(-1, 112)
        values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1, 112)
        b = masks.shape[0]
        if len(moves) != b:
            raise ValueError("one move list per position")
        priors_out, value_out = [], []
        for s in range(0, b, self.max_batch):
            e = min(b, s + self.max_batch)
            chunk = [np.asarray(m, dtype=np.int16).reshape(-1) for m in moves[s:e]]
            offsets = np.zeros(e - s + 1, np.int32)
            offsets[1:] = np.cumsum([c.size for c in chunk])
            idx = np.concatenate(chunk) if offsets[-1] else np.zeros(1, np.int16)
            priors = np.zeros(max(1, int(offsets[-1])), np.float32)
            value = np.zeros((e - s, 3 if self.wdl else 1), np.float32)
            _check(lib().mfh_net_eval_priors(self._h, e - s, _ptr(masks[s:e]), _ptr(values[s:e]),
                                             _ptr(offsets), _ptr(idx), float(softmax_temp),
                                             _ptr(priors), _ptr(value), None),
                   "mfh_net_eval_priors")
            priors_out += [priors[offsets[j]:offsets[j + 1]] for j in range(e - s)]
            value_out.append(value)
        return priors_out, np.concatenate(value_out)

    def eval_priors_flat(self, masks, values, offsets, indices, softmax_temp=1.0):
        """One mfh_net_eval_priors call on prepared arrays (batch <= max_batch):
        offsets int32 [B + 1], indices int16 [offsets[B]].  Returns (priors
        float32 [offsets[B]], raw value head output)."""
        b = masks.shape[0]
        priors = np.zeros(max(1, int(offsets[-1])), np.float32)
        value = np.zeros((b, 3 if self.wdl else 1), np.float32)
        _check(lib().mfh_net_eval_priors(self._h, b, _ptr(masks), _ptr(values), _ptr(offsets),
                                         _ptr(indices), float(softmax_temp), _ptr(priors),
                                         _ptr(value), None),
               "mfh_net_eval_priors")
        return priors[:int(offsets[-1])], value

    def eval_priors_device(self, batch, d_masks, d_values, d_offsets, d_indices, softmax_temp,
                           d_policy, d_priors, d_wdl, stream=None):
        """Device-resident form of eval_priors (pointers are device addresses)."""
        _check(lib().mfh_net_eval_priors_device(self._h, batch, d_masks, d_values, d_offsets,
                                                d_indices, float(softmax_temp), d_policy,
                                                d_priors, d_wdl, stream),
               "mfh_net_eval_priors_device")

    def evaluate_batch(self, planes):
        """NetworkOutput fields for planes [B,112,64] (EvaluateBatch)."""
        res = self.eval_planes(planes, with_moves_left=self.moves_left)
        policy, raw = res[0], res[1]
        if self.wdl:
            out = {"policy": policy, "wdl": raw, "value": raw[:, 0] - raw[:, 2]}
        else:
            out = {"policy": policy, "wdl": np.zeros((raw.shape[0], 3), np.float32),
                   "value": raw[:, 0]}
        if self.moves_left:
            out["moves_left"] = res[2]
        return out

    def evaluate(self, planes):
        out = self.evaluate_batch(np.asarray(planes).reshape(1, 112, 64))
        return {k: v[0] for k, v in out.items()}

    def eval_device(self, batch, d_masks, d_values, d_policy, d_wdl, stream=None):
        """Device-resident forward (pointers are device addresses)."""
        _check(lib().mfh_net_eval_device(self._h, batch, d_masks, d_values, d_policy, d_wdl,
                                         stream), "mfh_net_eval_device")

    def encoder_layer_ms(self, batch, layer, iterations, x_bits, x_lo_bits=None):
        """Runs body encoder layer `layer` alone `iterations` times on the
        residual stream x (bf16 bits [batch*64, E], x_lo_bits its lo plane in
        the split precisions) and returns milliseconds per run
        (mfh_debug_encoder_layer)."""
        x = np.ascontiguousarray(x_bits, dtype=np.uint16)
        lo = None if x_lo_bits is None else np.ascontiguousarray(x_lo_bits, dtype=np.uint16)
        ms = ctypes.c_float()
        _check(lib().mfh_debug_encoder_layer(self._h, batch, layer, iterations, _ptr(x),
                                             None if lo is None else _ptr(lo), ctypes.byref(ms)),
               "mfh_debug_encoder_layer")
        return ms.value

    def set_graphs(self, enabled: bool):
        """Graph capture/replay of the forward (on by default)."""
        _check(lib().mfh_net_set_graphs(self._h, 1 if enabled else 0), "mfh_net_set_graphs")

    def set_profiling(self, enabled: bool):
        _check(lib().mfh_net_set_profiling(self._h, 1 if enabled else 0), "mfh_net_set_profiling")

    def profile_reset(self):
        _check(lib().mfh_net_profile_reset(self._h), "mfh_net_profile_reset")

    def profile(self) -> dict:
        """{kernel kind: {launches, ms, flops, bytes}} accumulated since reset."""
        n = ctypes.c_int(0)
        _check(lib().mfh_net_profile(self._h, None, 0, ctypes.byref(n)), "mfh_net_profile")
        entries = (MfhProfileEntry * max(1, n.value))()
        _check(lib().mfh_net_profile(self._h, entries, n.value, ctypes.byref(n)),
               "mfh_net_profile")
        return {e.name.decode(): {"launches": e.launches, "ms": e.milliseconds,
                                  "flops": e.flops, "bytes": e.bytes}
                for e in entries[:n.value]}

    def debug_tensor(self, name, shape, dtype):
        out = np.zeros(shape, dtype=dtype)
        _check(lib().mfh_net_debug_tensor(self._h, name.encode(), out.ctypes.data, out.nbytes),
               "mfh_net_debug_tensor")
        return out


def pack_planes(planes):
    """Reference packed-input contract (input_plane_packing.h:61-83)."""
    planes = np.ascontiguousarray(planes, dtype=np.float32).reshape(-1, 112, 64)
    b = planes.shape[0]
    masks = np.zeros((b, 112), np.uint64)
    values = np.zeros((b, 112), np.float32)
    _check(lib().mfh_pack_planes(b, _ptr(planes), _ptr(masks), _ptr(values)), "mfh_pack_planes")
    return masks, values


def unpack_planes(masks, values):
    masks = np.ascontiguousarray(masks, dtype=np.uint64).reshape(-1, 112)
    values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1, 112)
    out = np.zeros((masks.shape[0], 112, 64), np.float32)
    _check(lib().mfh_debug_unpack_planes(masks.shape[0], _ptr(masks), _ptr(values), _ptr(out)),
           "mfh_debug_unpack_planes")
    return out


def quantize_fp8(w):
    """The library's host e4m3 row quantisation: (codes uint8, scales fp32)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows = w.shape[0]
    cols = w.size // rows
    codes = np.zeros((rows, cols), np.uint8)
    scale = np.zeros(rows, np.float32)
    _check(lib().mfh_debug_quantize_fp8(rows, cols, _ptr(w), _ptr(codes), _ptr(scale)),
           "mfh_debug_quantize_fp8")
    return codes, scale


def gemm_fp8(a_codes, ascale, w_codes, wscale, bias=None, act="none"):
    """fp8 x fp8 GEMM through mfh_debug_gemm_fp8 (a test hook): fp32
    act((A8.W8^T) * ascale[m] * wscale[n] + bias)."""
    a = np.ascontiguousarray(a_codes, dtype=np.uint8)
    w = np.ascontiguousarray(w_codes, dtype=np.uint8)
    sa = np.ascontiguousarray(ascale, dtype=np.float32)
    sw = np.ascontiguousarray(wscale, dtype=np.float32)
    m, k = a.shape
    n = w.shape[0]
    out = np.zeros((m, n), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    _check(lib().mfh_debug_gemm_fp8(m, n, k, _ptr(a), _ptr(sa), _ptr(w), _ptr(sw), _ptr(b),
                                    ACTIVATION[act], _ptr(out)), "mfh_debug_gemm_fp8")
    return out


def gemm_lo8(a_bits, a_lo8, w_bits, w_lo8, wscale, bias=None, act="none", bf16_out=False):
    """The BF16X2_FP8LO GEMM through mfh_debug_gemm_lo8 (a test hook):
    act((A.W^T + A_lo8.W_lo8^T) * wscale[n] + bias), bf16 bits and e4m3 codes
    as given.  fp32 output, or with ``bf16_out`` (hi bits, lo e4m3 codes of
    (out - hi) * 2^10)."""
    u16 = lambda x: np.ascontiguousarray(x, dtype=np.uint16)  # noqa: E731
    u8 = lambda x: np.ascontiguousarray(x, dtype=np.uint8)  # noqa: E731
    a, al, w, wl = u16(a_bits), u8(a_lo8), u16(w_bits), u8(w_lo8)
    sc = np.ascontiguousarray(wscale, dtype=np.float32)
    m, k = a.shape
    n = w.shape[0]
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    out = hi = lo = None
    if bf16_out:
        hi = np.zeros((m, n), np.uint16)
        lo = np.zeros((m, n), np.uint8)
    else:
        out = np.zeros((m, n), np.float32)
    _check(lib().mfh_debug_gemm_lo8(m, n, k, _ptr(a), _ptr(al), _ptr(w), _ptr(wl), _ptr(sc),
                                    _ptr(b), ACTIVATION[act], _ptr(out), _ptr(hi), _ptr(lo)),
           "mfh_debug_gemm_lo8")
    return (hi, lo) if bf16_out else out


def quantize_rows_e4m3(x_bits, x_lo_bits=None):
    """The device row quantiser (a test hook): (codes uint8, scales fp32)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    lo = None if x_lo_bits is None else np.ascontiguousarray(x_lo_bits, dtype=np.uint16)
    rows, cols = x.shape
    codes = np.zeros((rows, cols), np.uint8)
    scales = np.zeros(rows, np.float32)
    _check(lib().mfh_debug_quantize_rows_e4m3(rows, cols, _ptr(x), _ptr(lo), _ptr(codes),
                                              _ptr(scales)), "mfh_debug_quantize_rows_e4m3")
    return codes, scales


def gemm_bf16(a_bits, w_bits, bias=None, act="none"):
    a_bits = np.ascontiguousarray(a_bits, dtype=np.uint16)
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    m, k = a_bits.shape
    n = w_bits.shape[0]
    out = np.zeros((m, n), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    _check(lib().mfh_debug_gemm_bf16(m, n, k, _ptr(a_bits), _ptr(w_bits), _ptr(b),
                                     ACTIVATION[act], _ptr(out)), "mfh_debug_gemm_bf16")
    return out


def panel_gemm(a_bits, w_bits=None, a_lo_bits=None, w8_codes=None, wscale=None, bias=None,
               act="none", layernorm=None):
    """Row-panel GEMM through mfh_debug_panel_gemm (a test hook).  Without
    ``layernorm``: act(A.W^T + b) as (hi, lo) bf16 bit planes.  With
    ``layernorm`` = dict(gamma, beta, eps, alpha, resid32 | resid_hi +
    resid_lo): LN(resid + alpha (A.W^T + b)) as (hi, lo, fp32)."""
    u16 = lambda x: None if x is None else np.ascontiguousarray(x, dtype=np.uint16)
    f32 = lambda x: None if x is None else np.ascontiguousarray(x, dtype=np.float32)
    a_bits, a_lo_bits, w_bits = u16(a_bits), u16(a_lo_bits), u16(w_bits)
    w8 = None if w8_codes is None else np.ascontiguousarray(w8_codes, dtype=np.uint8)
    m, k = a_bits.shape
    n = (w_bits if w_bits is not None else w8).shape[0]
    hi = np.zeros((m, n), np.uint16)
    lo = np.zeros((m, n), np.uint16)
    ln = layernorm or {}
    y32 = np.zeros((m, n), np.float32) if layernorm is not None else None
    keep = [f32(wscale), f32(bias), f32(ln.get("resid32")), u16(ln.get("resid_hi")),
            u16(ln.get("resid_lo")), f32(ln.get("gamma")), f32(ln.get("beta"))]
    _check(lib().mfh_debug_panel_gemm(
        m, n, k, _ptr(a_bits), _ptr(a_lo_bits), _ptr(w_bits), _ptr(w8), _ptr(keep[0]),
        _ptr(keep[1]), ACTIVATION[act], 1 if layernorm is not None else 0, _ptr(keep[2]),
        _ptr(keep[3]), _ptr(keep[4]), float(ln.get("alpha", 1.0)), float(ln.get("eps", 1e-3)),
        _ptr(keep[5]), _ptr(keep[6]), _ptr(hi), _ptr(lo), _ptr(y32)), "mfh_debug_panel_gemm")
    return (hi, lo, y32) if layernorm is not None else (hi, lo)


def skinny_gemm(w_bits, a_bits=None, a_lo_bits=None, ln=None, bias=None, act="none",
                out_mode="bf16", resid=None, alpha=1.0, want_lo=False):
    """Few-row GEMM through mfh_debug_skinny_gemm (a test hook).  The A
    operand is the bf16 planes ``a_bits`` (+ ``a_lo_bits``), or ``ln`` =
    dict(x, gamma, beta, eps, rows, rows_per_src=1, split=True): the
    LayerNorm of fp32 source rows x.  ``out_mode`` "bf16" returns (hi, lo);
    "f32" and "resid" (``resid`` = fp32 array or (hi, lo) bit planes) return
    (out, stats [parts, M, 2]); with ``ln`` the normalised rows (hi, lo, fp32)
    come last."""
    u16 = lambda x: None if x is None else np.ascontiguousarray(x, dtype=np.uint16)
    f32 = lambda x: None if x is None else np.ascontiguousarray(x, dtype=np.float32)
    w_bits = u16(w_bits)
    n, k = w_bits.shape
    a_bits, a_lo_bits = u16(a_bits), u16(a_lo_bits)
    m = a_bits.shape[0] if a_bits is not None else int(ln["rows"])
    mode = {"bf16": 0, "f32": 1, "resid": 2}[out_mode]
    out = np.zeros((m, n), np.uint16 if mode == 0 else np.float32)
    out_lo = np.zeros((m, n), np.uint16) if mode == 0 and want_lo else None
    stats = np.zeros((max(1, (n + 15) // 16), m, 2), np.float32) if mode else None
    parts = ctypes.c_int(0)
    ln = ln or {}
    rps = int(ln.get("rows_per_src", 1))
    y = [np.zeros((m, k), t) for t in (np.uint16, np.uint16, np.float32)] if ln and rps == 1 \
        else [None, None, None]
    r32 = rh = rl = None
    if mode == 2:
        if isinstance(resid, tuple):
            rh, rl = u16(resid[0]), u16(resid[1])
        else:
            r32 = f32(resid)
    keep = [f32(ln.get("x")), f32(ln.get("gamma")), f32(ln.get("beta")), f32(bias)]
    _check(lib().mfh_debug_skinny_gemm(
        m, n, k, _ptr(a_bits), _ptr(a_lo_bits), _ptr(keep[0]), rps, float(ln.get("eps", 1e-3)),
        _ptr(keep[1]), _ptr(keep[2]), 1 if ln.get("split", True) else 0, _ptr(w_bits),
        _ptr(keep[3]), ACTIVATION[act], mode, _ptr(r32), _ptr(rh), _ptr(rl), float(alpha),
        _ptr(out), _ptr(out_lo), _ptr(stats), ctypes.byref(parts), _ptr(y[0]), _ptr(y[1]),
        _ptr(y[2])), "mfh_debug_skinny_gemm")
    res = (out, out_lo) if mode == 0 else (out, stats[:parts.value])
    return res + (tuple(y),) if ln and rps == 1 else res


def create_network(spec, weights, max_batch=256, device=-1, precision="bf16x2",
                   weights_dtype="bf16", fused_layernorm=False):
    """HipNetwork for a synth.NetSpec and its weights.  ``precision`` is
    "bf16x2" (split activations, default: meets every parity gate),
    "bf16x2_gemm" or "bf16" (single-pass, twice the MFMA throughput), or
    "fp8" (e4m3 activations; experimental, below the parity gates, refused
    unless METALFISH_HIP_EXPERIMENTAL_FP8=1);
    ``weights_dtype`` "bf16" or "fp8" (e4m3 with per-row scales);
    ``fused_layernorm`` selects the row-panel residual GEMM + LayerNorm."""
    return HipNetwork(weights, spec.heads, wdl=spec.wdl, moves_left=spec.moves_left_dim > 0,
                      pe_map=spec.pe_map, pol_heads=spec.policy_heads,
                      default_activation=spec.default_activation,
                      ffn_activation=spec.ffn_activation,
                      smolgen_activation=spec.smolgen_activation, max_batch=max_batch,
                      device=device, precision=precision, weights_dtype=weights_dtype,
                      fused_layernorm=fused_layernorm)


class WeightsFile:
    """A decoded network file: the NetworkFormat after the reference's legacy
    fix-ups (``format``), head counts and the weight inventory of the
    selected heads (``tensors`` {name: fp32 array}, ``dims``) -- LoadWeights,
    MultiHeadWeights and CreateNetworkWeightInventory of the reference
    (src/nn/loader.cpp:162-189, src/nn/weights.cpp:216-291,
    src/nn/network_weight_inventory.cpp:332-352)."""

    def __init__(self, handle):
        L = lib()
        try:
            fmt = MfhWeightsFormat()
            _check(L.mfh_weights_describe(handle, ctypes.byref(fmt), None),
                   "mfh_weights_describe")
            self.format = {k: getattr(fmt, k) for k in FORMAT_FIELDS}
            self.headcount = fmt.headcount
            self.pol_headcount = fmt.pol_headcount
            views = ctypes.POINTER(MfhTensor)()
            n = ctypes.c_int(0)
            _check(L.mfh_weights_tensors(handle, ctypes.byref(views), ctypes.byref(n)),
                   "mfh_weights_tensors")
            self.tensors, self.dims = {}, {}
            for j in range(n.value):
                t = views[j]
                name = t.name.decode()
                buf = (ctypes.c_float * t.count).from_address(t.data)
                self.tensors[name] = np.frombuffer(buf, dtype=np.float32).copy()
                d = ctypes.POINTER(ctypes.c_uint32)()
                nd = ctypes.c_int(0)
                _check(L.mfh_weights_tensor_dims(handle, j, ctypes.byref(d), ctypes.byref(nd)),
                       "mfh_weights_tensor_dims")
                self.dims[name] = [d[k] for k in range(nd.value)]
        finally:
            L.mfh_weights_free(handle)

    def create_network(self, max_batch=256, device=-1, precision="bf16x2",
                       weights_dtype="bf16"):
        """HipNetwork for this file (CreateNetwork(const WeightsFile&, ...),
        reference src/nn/network.cpp:137-208)."""
        return HipNetwork(self.tensors, self.headcount, max_batch=max_batch, device=device,
                          precision=precision, weights_dtype=weights_dtype,
                          net_format=self.format, pol_heads=self.pol_headcount)


def load_weights(path) -> WeightsFile:
    """Reads a ``.pb`` / ``.pb.gz`` network file (no device needed)."""
    h = ctypes.c_void_p()
    _check(lib().mfh_weights_load(os.fsencode(path), ctypes.byref(h)), "mfh_weights_load")
    return WeightsFile(h)


def parse_weights(data: bytes) -> WeightsFile:
    """Decodes a serialised Net message held in memory."""
    h = ctypes.c_void_p()
    buf = ctypes.create_string_buffer(bytes(data), len(data))
    _check(lib().mfh_weights_parse(buf, len(data), ctypes.byref(h)), "mfh_weights_parse")
    return WeightsFile(h)
