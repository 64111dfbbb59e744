"""Hand-built nets of the reference CPU backend's known-answer tests.

Each builder rebuilds the weights of one ``make_*_cpu_weights_file`` in
reference ``tests/test_mcts_module.cpp:142-505``; the expected outputs are the
values asserted in ``test_cpu_backend_*`` (``test_mcts_module.cpp:2483-2651``).
Tensor names follow the reference's weight inventory (``body.ip_emb_w``,
``policy.vanilla.ip_pol_w``, ...) and every matrix is ``[out][in]``.
"""

import numpy as np

from oracle.plan import NetFormat

P = 112  # packed input planes
S = 64   # squares
POLICY = 1858


def _z(*shape):
    return np.zeros(shape, dtype=np.float32)


def dense_only():
    """make_dense_only_cpu_weights_file (test_mcts_module.cpp:142-180)."""
    fmt = NetFormat(attention_body=False, attention_policy=False, wdl=False,
                    input_embedding="NONE", default_activation="relu", ffn_activation="relu",
                    smolgen_activation="relu")
    pb = _z(POLICY)
    pb[0], pb[10] = 1.25, 0.5
    t = {"policy.vanilla.ip_pol_w": _z(POLICY, P), "policy.vanilla.ip_pol_b": pb,
         "value.winner.ip_val_w": _z(1, P), "value.winner.ip_val_b": np.array([0.25], np.float32)}
    expect = {"policy": {0: 1.25, 10: 0.5}, "value": 0.25, "tol": 1e-6}
    return fmt, t, _z(112, 64), expect


def gate_ffn():
    """make_gate_ffn_cpu_weights_file (test_mcts_module.cpp:182-245)."""
    fmt = NetFormat(attention_body=False, attention_policy=False, wdl=False,
                    input_embedding="NONE", default_activation="relu", ffn_activation="relu",
                    smolgen_activation="relu")
    eye = np.eye(2, dtype=np.float32)
    pw = _z(POLICY, 2)
    pw[0, 0] = 1.0
    pw[10, 1] = 1.0
    t = {"body.ip_emb_w": _z(2, P), "body.ip_emb_b": np.array([1.0, 2.0], np.float32),
         "body.ip_mult_gate": np.array([2.0, 3.0], np.float32),
         "body.ip_add_gate": np.array([1.0, -1.0], np.float32),
         "body.ip_emb_ffn.dense1_w": eye.copy(), "body.ip_emb_ffn.dense1_b": _z(2),
         "body.ip_emb_ffn.dense2_w": eye.copy(),
         "body.ip_emb_ffn.dense2_b": np.array([1.0, -1.0], np.float32),
         "body.ip_emb_ffn_ln_gammas": np.ones(2, np.float32),
         "body.ip_emb_ffn_ln_betas": _z(2),
         "policy.vanilla.ip_pol_w": pw, "policy.vanilla.ip_pol_b": _z(POLICY),
         "value.winner.ip_val_w": _z(1, 2), "value.winner.ip_val_b": np.array([0.75], np.float32)}
    # policy[0] in (-1.01, -0.99), policy[10] in (0.99, 1.01), value 0.75 +- 1e-6
    expect = {"policy_range": {0: (-1.01, -0.99), 10: (0.99, 1.01)}, "value": 0.75, "tol": 1e-6}
    return fmt, t, _z(112, 64), expect


def positional_metadata():
    """make_positional_metadata_cpu_weights_file (test_mcts_module.cpp:247-290)."""
    fmt = NetFormat(attention_body=False, attention_policy=False, wdl=False,
                    input_embedding="NONE", default_activation="relu", ffn_activation="relu",
                    smolgen_activation="relu")
    pw = _z(POLICY, 2)
    pw[0, 0] = 1.0
    pw[10, 1] = 1.0
    t = {"body.ip_emb_w": _z(2, P), "body.ip_emb_b": np.array([0.25, 0.5], np.float32),
         "body.smolgen_w": _z(S * S),
         "policy.vanilla.ip_pol_w": pw, "policy.vanilla.ip_pol_b": _z(POLICY),
         "value.winner.ip_val_w": _z(1, 2), "value.winner.ip_val_b": np.array([0.5], np.float32)}
    expect = {"policy": {0: 0.25, 10: 0.5}, "value": 0.5, "tol": 1e-6}
    return fmt, t, _z(112, 64), expect


def dynamic_pe():
    """make_dynamic_pe_cpu_weights_file (test_mcts_module.cpp:292-360)."""
    fmt = NetFormat(attention_body=False, attention_policy=False, wdl=False,
                    input_embedding="PE_DENSE", default_activation="relu",
                    ffn_activation="relu", smolgen_activation="relu")
    pe_w, emb_w = 1, 2
    flat = S * emb_w
    pos_in, pos_out, concat = 12 * S, pe_w * S, P + pe_w
    pre_w = _z(pos_out, pos_in)
    pre_b = _z(pos_out)
    for sq in range(S):
        pre_w[sq, sq * 12 + 0] = 0.25
        pre_w[sq, sq * 12 + 11] = 0.5
        pre_b[sq] = np.float32(0.01) * np.float32(sq)
    ew = _z(emb_w, concat)
    ew[0, 0] = 1.0
    ew[0, P] = 1.0
    ew[1, 12] = np.float32(0.10)
    pw = _z(POLICY, flat)
    pw[0, 0] = 1.0
    pw[10, 5 * emb_w + 0] = 1.0
    vw = _z(1, flat)
    vw[0, 1] = 1.0
    t = {"body.ip_emb_preproc_w": pre_w, "body.ip_emb_preproc_b": pre_b,
         "body.ip_emb_w": ew, "body.ip_emb_b": _z(emb_w),
         "policy.vanilla.ip_pol_w": pw, "policy.vanilla.ip_pol_b": _z(POLICY),
         "value.winner.ip_val_w": vw, "value.winner.ip_val_b": _z(1)}
    planes = _z(112, 64)
    planes[0, 0] = 2.0
    planes[0, 5] = 2.0
    planes[11, 0] = -1.5
    planes[12, 0] = 7.0
    expect = {"policy": {0: 1.75, 10: 2.55}, "value": 0.70, "tol": 1e-5}
    return fmt, t, planes, expect


def attention():
    """make_attention_cpu_weights_file (test_mcts_module.cpp:362-430)."""
    fmt = NetFormat(attention_body=True, attention_policy=False, wdl=False,
                    input_embedding="PE_DENSE", default_activation="relu",
                    ffn_activation="relu", smolgen_activation="relu", body_heads=1)
    emb_w = 2
    flat = S * emb_w
    concat = P + 1
    ew = _z(emb_w, concat)
    ew[0, 0] = 1.0
    ew[1, 1] = 1.0
    eye = np.eye(2, dtype=np.float32)
    pw = _z(POLICY, flat)
    pw[0, 0] = 1.0
    pw[1, 1] = 1.0
    vw = _z(1, flat)
    vw[0, 1] = 1.0
    m = "body.encoder.0.mha."
    t = {"body.ip_emb_preproc_w": _z(S, 12 * S), "body.ip_emb_preproc_b": _z(S),
         "body.ip_emb_w": ew, "body.ip_emb_b": _z(emb_w),
         m + "q_w": _z(2, 2), m + "q_b": _z(2), m + "k_w": _z(2, 2), m + "k_b": _z(2),
         m + "v_w": eye.copy(), m + "v_b": _z(2), m + "dense_w": eye.copy(), m + "dense_b": _z(2),
         "policy.vanilla.ip_pol_w": pw, "policy.vanilla.ip_pol_b": _z(POLICY),
         "value.winner.ip_val_w": vw, "value.winner.ip_val_b": _z(1)}
    planes = _z(112, 64)
    planes[0, 0] = 2.0
    planes[1, 1] = 4.0
    expect = {"policy": {0: 2.0 / 64.0, 1: 4.0 / 64.0}, "value": 4.0 / 64.0, "tol": 1e-5}
    return fmt, t, planes, expect


def attention_policy_map():
    """make_attention_policy_cpu_weights_file (test_mcts_module.cpp:432-505)."""
    fmt = NetFormat(attention_body=True, attention_policy=True, wdl=False,
                    input_embedding="PE_DENSE", default_activation="relu",
                    ffn_activation="relu", smolgen_activation="relu")
    body_w = 2
    flat = S * body_w
    concat = P + 1
    bw = _z(body_w, concat)
    bw[0, 0] = 1.0
    bw[1, 1] = 1.0
    vw = _z(1, flat)
    vw[0, 0] = 1.0
    pp = "policy.vanilla."
    t = {"body.ip_emb_preproc_w": _z(S, 12 * S), "body.ip_emb_preproc_b": _z(S),
         "body.ip_emb_w": bw, "body.ip_emb_b": _z(body_w),
         pp + "ip_pol_w": np.eye(2, dtype=np.float32), pp + "ip_pol_b": _z(2),
         pp + "ip2_pol_w": np.array([[1.0, 0.0]], np.float32), pp + "ip2_pol_b": _z(1),
         pp + "ip3_pol_w": np.array([[0.0, 1.0]], np.float32), pp + "ip3_pol_b": _z(1),
         pp + "ip4_pol_w": np.array([[1.0], [3.0], [5.0], [0.0]], np.float32),
         "value.winner.ip_val_w": vw, "value.winner.ip_val_b": _z(1)}
    planes = _z(112, 64)
    planes[0, 0] = 2.0
    planes[1, 1] = 5.0
    planes[0, 48] = 2.0
    planes[1, 56] = 7.0
    expect = {"policy": {0: 10.0, 1793: 15.0}, "value": 2.0, "tol": 1e-5}
    return fmt, t, planes, expect


ALL = {
    "dense_only": dense_only,
    "gate_ffn": gate_ffn,
    "positional_metadata": positional_metadata,
    "dynamic_pe": dynamic_pe,
    "attention": attention,
    "attention_policy_map": attention_policy_map,
}
