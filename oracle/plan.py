"""CPU ORACLE -- TEST INFRASTRUCTURE ONLY.

Restates how MetalFish's reference CPU backend turns a weights file into an
ordered list of steps and wires their inputs and outputs, so that
``cpu_ref.c`` (the numerics) can execute them.  Only tests/,
``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may import this
package, and only as the checker; the product (``metalfish_amd``) never does.

Sources restated (all paths under the reference tree):

* step order -- ``src/nn/network_execution_plan.cpp:94-223`` (AddBody,
  AddPolicy, AddValue, AddMovesLeft) and ``681-700`` (CreateNetworkExecutionPlan);
* dense-stage activations -- ``network_execution_plan.cpp:1080-1119``;
* residual scale alpha = (2L)^-1/4 -- ``network_execution_plan.cpp:1152-1162``;
* LayerNorm epsilons -- ``network_execution_plan.cpp:1164-1193``;
* head counts -- ``network_execution_plan.cpp:1023-1030``;
* data flow (source_for / remember_output / residual parents / step
  skipping) -- ``src/nn/cpu/cpu_network.cpp:580-690, 1399-1457``;
* output decode -- ``cpu_network.cpp:1460-1490`` and
  ``src/nn/network_output_decoder.cpp:31-78`` (value = W - L).

Parity pinning (what fixes each part independently of this restatement):

* dense / gate / FFN / positional / dynamic PE / attention / attention policy
  map: the reference's CPU known-answer tests
  (``tests/test_mcts_module.cpp:142-505, 2483-2651``), rebuilt in
  ``tests/test_oracle_kat.py``;
* LayerNorm, softmax, activations, smolgen, attention with bias, the
  promotion-logit formula and alpha/eps rules: closed forms and brute-force
  float64 recomputation on small random nets in ``tests/test_oracle_math.py``;
* attention-policy gather table: bit-exact against the reference's
  ``kAttnPolicyMap`` (``tests/test_policy_tables.py``);
* input packing: the start-position fixture
  (``tests/nn_input_fixture.h:39-58``) in ``tests/test_inputs.py``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .policy_tables import pos_encoding

DENSE, LAYERNORM, GATE, FFN, ATTENTION, POLICY_MAP, DYNAMIC_PE, STATIC_PE = 1, 2, 3, 4, 5, 6, 7, 8

ACTIVATIONS = {
    "": -1,
    "relu": 0,
    "relu_2": 1,
    "tanh": 2,
    "sigmoid": 3,
    "swish": 4,
    "mish": 5,
    "selu": 6,
    "softmax": 7,
}

MAX_TENSORS = 24


class OrStep(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int),
        ("src", ctypes.c_int),
        ("dst", ctypes.c_int),
        ("parent", ctypes.c_int),
        ("act", ctypes.c_int),
        ("alpha", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("heads", ctypes.c_int),
        ("aux0", ctypes.c_int),
        ("aux1", ctypes.c_int),
        ("n_tensors", ctypes.c_int),
        ("t", ctypes.c_void_p * MAX_TENSORS),
        ("d0", ctypes.c_int * MAX_TENSORS),
        ("d1", ctypes.c_int * MAX_TENSORS),
        ("tag", ctypes.c_int * MAX_TENSORS),
    ]


@dataclass
class NetFormat:
    """Network format descriptor (reference ``network_format.cpp:72-127``)."""

    attention_body: bool = True
    attention_policy: bool = True
    wdl: bool = True
    moves_left: bool = False
    input_embedding: str = "PE_DENSE"  # "PE_DENSE", "PE_MAP" or "NONE"
    default_activation: str = "mish"
    ffn_activation: str = "mish"
    smolgen_activation: str = "swish"
    body_heads: int = 0
    policy_heads: int = 0


@dataclass
class PlanStep:
    kind: str  # input_pack, dense, layernorm, gate, ffn, attention,
    #            positional, policy_map, output_decode
    name: str
    tensors: list = field(default_factory=list)


def _add_if_any(steps, present, kind, name, tensor_names):
    names = [t for t in tensor_names if t in present]
    if names:
        steps.append(PlanStep(kind, name, names))


def _has_prefix(present, prefix):
    return any(t.startswith(prefix) for t in present)


def _add_encoder_series(steps, present, prefix, name):
    i = 0
    while _has_prefix(present, f"{prefix}.{i}."):
        lp, ln = f"{prefix}.{i}", f"{name}.{i}"
        mha = lp + ".mha"
        _add_if_any(steps, present, "attention", ln + ".mha",
                    [mha + s for s in (".q_w", ".q_b", ".k_w", ".k_b", ".v_w", ".v_b",
                                       ".dense_w", ".dense_b")])
        sg = mha + ".smolgen"
        _add_if_any(steps, present, "dense", ln + ".mha.smolgen.dense",
                    [sg + s for s in (".compress", ".dense1_w", ".dense1_b", ".dense2_w",
                                      ".dense2_b")])
        _add_if_any(steps, present, "layernorm", ln + ".mha.smolgen.norm",
                    [sg + s for s in (".ln1_gammas", ".ln1_betas", ".ln2_gammas",
                                      ".ln2_betas")])
        _add_if_any(steps, present, "layernorm", ln + ".ln1",
                    [lp + ".ln1_gammas", lp + ".ln1_betas"])
        _add_if_any(steps, present, "ffn", ln + ".ffn",
                    [lp + ".ffn" + s for s in (".dense1_w", ".dense1_b", ".dense2_w",
                                               ".dense2_b")])
        _add_if_any(steps, present, "layernorm", ln + ".ln2",
                    [lp + ".ln2_gammas", lp + ".ln2_betas"])
        i += 1


def build_plan(fmt: NetFormat, present, policy_head="vanilla", value_head="winner"):
    """Ordered step list (reference network_execution_plan.cpp:94-223, 681-700)."""
    steps = [PlanStep("input_pack", "input.pack")]
    dense = lambda p, n: _add_if_any(steps, present, "dense", n, [p + "_w", p + "_b"])
    norm = lambda p, n: _add_if_any(steps, present, "layernorm", n,
                                    [p + "_gammas", p + "_betas"])
    conv = lambda p, n: _add_if_any(steps, present, "convolution", n,
                                    [p + ".weights", p + ".biases"])
    ffn = lambda p, n: _add_if_any(steps, present, "ffn", n,
                                   [p + s for s in (".dense1_w", ".dense1_b", ".dense2_w",
                                                    ".dense2_b")])
    # AddBody
    conv("body.input", "body.input")
    dense("body.ip_emb_preproc", "body.input_embedding_preprocess")
    dense("body.ip_emb", "body.input_embedding")
    norm("body.ip_emb_ln", "body.input_embedding_norm")
    _add_if_any(steps, present, "gate", "body.input_embedding_gates",
                ["body.ip_mult_gate", "body.ip_add_gate"])
    ffn("body.ip_emb_ffn", "body.input_embedding_ffn")
    norm("body.ip_emb_ffn_ln", "body.input_embedding_ffn_norm")
    _add_if_any(steps, present, "positional", "body.smolgen_positional", ["body.smolgen_w"])
    _add_encoder_series(steps, present, "body.encoder", "body.encoder")
    if _has_prefix(present, "body.residual."):
        steps.append(PlanStep("convolution", "body.residual"))
    # AddMovesLeft
    if fmt.moves_left:
        conv("moves_left", "moves_left.conv")
        dense("moves_left.ip_mov", "moves_left.dense0")
        dense("moves_left.ip1_mov", "moves_left.dense1")
        dense("moves_left.ip2_mov", "moves_left.output")
    # AddPolicy
    pp = f"policy.{policy_head}"
    conv(pp + ".policy1", pp + ".policy1")
    conv(pp + ".policy", pp + ".policy")
    _add_encoder_series(steps, present, pp + ".encoder", pp + ".encoder")
    dense(pp + ".ip_pol", pp + ".output")
    dense(pp + ".ip2_pol", pp + ".dense2")
    dense(pp + ".ip3_pol", pp + ".dense3")
    _add_if_any(steps, present, "policy_map", pp + ".policy_map", [pp + ".ip4_pol_w"])
    # AddValue
    vp = f"value.{value_head}"
    conv(vp + ".value", vp + ".value")
    dense(vp + ".ip_val", vp + ".output")
    dense(vp + ".ip1_val", vp + ".dense1")
    dense(vp + ".ip2_val", vp + ".dense2")
    dense(vp + ".ip_val_err", vp + ".error")
    steps.append(PlanStep("output_decode", "output.decode"))
    return steps


def encoder_layer_count(steps):
    """NetworkBodyEncoderLayerCount (network_execution_plan.cpp:1121-1150)."""
    n = 0
    for s in steps:
        if s.name.startswith("body.encoder."):
            head = s.name[len("body.encoder."):].split(".", 1)[0]
            if head.isdigit():
                n = max(n, int(head) + 1)
    return n


def residual_scale(steps, stage):
    """NetworkFeedForwardResidualScale (network_execution_plan.cpp:1152-1162)."""
    if not (stage.startswith("body.input_embedding_ffn") or stage.startswith("body.encoder.")):
        return np.float32(1.0)
    n = encoder_layer_count(steps)
    if n == 0:
        return np.float32(1.0)
    return np.float32(_lib.powf(np.float32(2.0) * np.float32(n), np.float32(-0.25)))


def ffn_ln_eps(fmt, stage):
    """NetworkFeedForwardLayerNormEpsilon (network_execution_plan.cpp:1164-1173)."""
    if stage.startswith("body.input_embedding_ffn"):
        return np.float32(1e-3)
    if stage.startswith("body.encoder."):
        return np.float32(1e-3) if fmt.input_embedding == "PE_DENSE" else np.float32(1e-6)
    return np.float32(1e-5)


def dense_ln_eps(fmt, stage):
    """NetworkDenseLayerNormEpsilon (network_execution_plan.cpp:1175-1182)."""
    if stage == "body.input_embedding_norm" and fmt.input_embedding == "PE_DENSE":
        return np.float32(1e-3)
    return np.float32(1e-5)


def attention_ln_eps(fmt, stage):
    """NetworkAttentionLayerNormEpsilon (network_execution_plan.cpp:1184-1193)."""
    if stage.startswith("body.encoder."):
        return np.float32(1e-3) if fmt.input_embedding == "PE_DENSE" else np.float32(1e-6)
    if stage.startswith("policy."):
        return np.float32(1e-6)
    return np.float32(1e-5)


def dense_activation(fmt, policy_head, value_head, stage):
    """NetworkDenseStageActivationName (network_execution_plan.cpp:1080-1119)."""
    pp, vp = f"policy.{policy_head}.", f"value.{value_head}."
    if stage.startswith(pp):
        if stage in (pp + "dense2", pp + "dense3"):
            return ""
        if stage == pp + "output":
            if not fmt.attention_policy:
                return ""
            return fmt.default_activation if fmt.attention_body else "selu"
    if stage.startswith(vp):
        if stage == vp + "dense2":
            return "softmax" if fmt.wdl else "tanh"
        if stage in (vp + "output", vp + "dense1"):
            return fmt.default_activation
    if stage == "moves_left.output":
        return "relu"
    if stage in ("moves_left.dense0", "moves_left.dense1"):
        return fmt.default_activation
    if stage == "body.input_embedding_preprocess":
        return ""
    if stage == "body.input_embedding":
        return fmt.default_activation
    return fmt.ffn_activation


def head_count(fmt, stage):
    if stage.startswith("body.encoder."):
        return fmt.body_heads
    if stage.startswith("policy."):
        return fmt.policy_heads
    return 0


class ResolvedProgram:
    """Steps lowered to ``OrStep`` records plus buffer bookkeeping."""

    def __init__(self, fmt: NetFormat, tensors: dict, policy_head="vanilla",
                 value_head="winner", gather=None):
        self.fmt = fmt
        self.tensors = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in tensors.items()}
        self.policy_head, self.value_head = policy_head, value_head
        self.plan = build_plan(fmt, set(self.tensors), policy_head, value_head)
        self._keep = []
        self.records = []
        self._lower(gather)

    def _tensor(self, rec, slot, name, tag=0):
        arr = self.tensors[name]
        rec.t[slot] = arr.ctypes.data
        rec.d0[slot] = arr.shape[0]
        rec.d1[slot] = arr.shape[1] if arr.ndim == 2 else 0
        rec.tag[slot] = tag
        rec.n_tensors = max(rec.n_tensors, slot + 1)

    def _lower(self, gather):
        fmt, steps = self.fmt, self.plan
        for s in steps:
            if s.kind == "convolution":
                raise ValueError("CPU transformer backend does not support convolution yet: "
                                 + s.name)
        pp, vp = f"policy.{self.policy_head}.", f"value.{self.value_head}."
        outputs = {}
        nbuf = [1]  # buffer 0 = packed plane values
        last = {"body": None, "policy": None, "value": None, "moves": None}
        last_executed = last_ffn = last_attention = None
        ffn_src, attn_src, attn_policy_src = {}, {}, {}

        def new_buf():
            nbuf[0] += 1
            return nbuf[0] - 1

        def source_for(name):
            if name.startswith(pp):
                if fmt.attention_policy and name == pp + "dense3" and pp in attn_policy_src:
                    return attn_policy_src[pp]
                return outputs[last["policy"]] if last["policy"] else (
                    outputs[last["body"]] if last["body"] else 0)
            if name.startswith(vp):
                return outputs[last["value"]] if last["value"] else (
                    outputs[last["body"]] if last["body"] else 0)
            if name.startswith("moves_left."):
                return outputs[last["moves"]] if last["moves"] else (
                    outputs[last["body"]] if last["body"] else 0)
            return outputs[last["body"]] if last["body"] else 0

        def remember(name, buf):
            outputs[name] = buf
            if name.startswith(pp):
                last["policy"] = name
            elif name.startswith(vp):
                last["value"] = name
            elif name.startswith("moves_left."):
                last["moves"] = name
            elif name.startswith("body."):
                last["body"] = name

        by_name = {s.name: s for s in steps}
        global_step = next((s for s in steps if s.kind == "positional"), None)

        for s in steps:
            if s.kind in ("input_pack", "output_decode"):
                continue
            if (s.kind == "dense" and s.name.endswith(".mha.smolgen.dense")) or (
                    s.kind == "layernorm" and s.name.endswith(".mha.smolgen.norm")):
                continue  # consumed inside the attention stage, not "executed"
            rec = OrStep()
            rec.parent = -1
            if s.kind == "dense" and s.name == "body.input_embedding_preprocess":
                if fmt.input_embedding != "PE_DENSE":
                    raise ValueError("CPU dynamic PE tensor plan is invalid: " + s.name)
                rec.kind, rec.src, rec.dst = DYNAMIC_PE, 0, new_buf()
                self._tensor(rec, 0, s.tensors[0])
                self._tensor(rec, 1, s.tensors[1])
                self.records.append(rec)
                remember(s.name, rec.dst)
                last_executed = s.name
                continue
            if (s.kind == "dense" and s.name == "body.input_embedding"
                    and fmt.input_embedding == "PE_MAP" and fmt.attention_body
                    and last["body"] is None):
                # PE_MAP: planes concatenated with the static position
                # encoding feed the embedding dense (the CUDA backend's
                # StaticPositionEncodingConcatKernel, cuda_kernels.cu:1016-1040,
                # for IsStaticPositionEmbeddingStage, cuda_stage_executor.cpp:
                # 487-492; width = ip_emb_w in-dim - 112,
                # network_execution_plan.cpp:833-865).
                pe = np.ascontiguousarray(pos_encoding(), dtype=np.float32)
                pe_w = self.tensors[s.tensors[0]].shape[1] - 112
                if pe_w != pe.shape[1]:
                    raise ValueError("static position encoding width mismatch")
                self._keep.append(pe)
                pre = OrStep()
                pre.parent = -1
                pre.kind, pre.src, pre.dst = STATIC_PE, 0, new_buf()
                pre.t[0] = pe.ctypes.data
                pre.d0[0], pre.d1[0] = pe.shape[0], pe.shape[1]
                pre.n_tensors = 1
                self.records.append(pre)
                remember("body.input_embedding_static_pe", pre.dst)
            src = source_for(s.name)
            if s.kind == "positional":
                last_executed = s.name
                continue
            if s.kind == "dense":
                if fmt.attention_policy and s.name == pp + "dense2":
                    attn_policy_src[pp] = src
                rec.kind, rec.src, rec.dst = DENSE, src, new_buf()
                rec.act = ACTIVATIONS[dense_activation(fmt, self.policy_head,
                                                       self.value_head, s.name)]
                self._tensor(rec, 0, s.tensors[0])
                self._tensor(rec, 1, s.tensors[1])
            elif s.kind == "policy_map":
                if not fmt.attention_policy:
                    raise ValueError("CPU transformer backend does not support policy "
                                     "mapping yet: " + s.name)
                prefix = s.name[: -len(".policy_map")]
                rec.kind, rec.src, rec.dst = POLICY_MAP, src, new_buf()
                rec.aux0 = outputs[prefix + ".dense2"]
                rec.aux1 = outputs[prefix + ".dense3"]
                self._tensor(rec, 0, s.tensors[0])
                g = np.ascontiguousarray(gather, dtype=np.float32)
                self._keep.append(g)
                rec.t[1] = g.ctypes.data
                rec.d0[1], rec.d1[1] = g.shape[0], 0
                rec.n_tensors = 2
            elif s.kind == "attention":
                rec.kind, rec.src, rec.dst = ATTENTION, src, new_buf()
                rec.heads = head_count(fmt, s.name)
                rec.act = ACTIVATIONS[fmt.smolgen_activation]
                for i, t in enumerate(s.tensors):
                    self._tensor(rec, i, t)
                sd, sn = by_name.get(s.name + ".smolgen.dense"), by_name.get(
                    s.name + ".smolgen.norm")
                if sd is not None:
                    if sn is None or global_step is None:
                        raise ValueError("CPU attention smolgen requires global positional "
                                         "weights: " + s.name)
                    for i, t in enumerate(sd.tensors + sn.tensors):
                        self._tensor(rec, 8 + i, t)
                    self._tensor(rec, 17, global_step.tensors[0])
                attn_src[s.name] = src
                last_attention = s.name
            elif s.kind == "gate":
                rec.kind, rec.src, rec.dst = GATE, src, new_buf()
                for i, t in enumerate(s.tensors):
                    self._tensor(rec, i, t, tag=1 if "mult_gate" in t else 2)
            elif s.kind == "ffn":
                rec.kind, rec.src, rec.dst = FFN, src, new_buf()
                rec.act = ACTIVATIONS[fmt.ffn_activation]
                for i, t in enumerate(s.tensors):
                    self._tensor(rec, i, t)
                ffn_src[s.name] = src
                last_ffn = s.name
            elif s.kind == "layernorm":
                rec.kind, rec.src, rec.dst = LAYERNORM, src, new_buf()
                self._tensor(rec, 0, s.tensors[0])
                self._tensor(rec, 1, s.tensors[1])
                rec.alpha, rec.eps = 1.0, dense_ln_eps(fmt, s.name)
                if last_ffn is not None and last_executed == last_ffn:
                    rec.parent = ffn_src[last_ffn]
                    rec.alpha = residual_scale(steps, last_ffn)
                    rec.eps = ffn_ln_eps(fmt, last_ffn)
                elif last_attention is not None and last_executed == last_attention:
                    rec.parent = attn_src[last_attention]
                    rec.alpha = residual_scale(steps, s.name)
                    rec.eps = attention_ln_eps(fmt, s.name)
            else:
                raise ValueError(f"CPU transformer backend does not support {s.kind} yet: "
                                 + s.name)
            self.records.append(rec)
            remember(s.name, rec.dst)
            last_executed = s.name

        self.n_buffers = nbuf[0]
        pol = pp + "policy_map" if pp + "policy_map" in outputs else pp + "output"
        if vp + "dense2" in outputs:
            val = vp + "dense2"
        elif vp + "output" in outputs:
            val = vp + "output"
        else:
            val = last["value"]
        self.policy_buf = outputs[pol]
        self.value_buf = outputs[val]
        self.moves_buf = -1
        if fmt.moves_left:
            mv = "moves_left.output" if "moves_left.output" in outputs else last["moves"]
            self.moves_buf = outputs[mv]
        self.policy_width = 1858
        self.value_width = 3 if fmt.wdl else 1
        arr = (OrStep * len(self.records))(*self.records)
        self.c_steps = arr
