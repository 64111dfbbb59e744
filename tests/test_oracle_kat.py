"""The reference CPU backend's known-answer tests, run against the oracle.

Nets and expectations: reference tests/test_mcts_module.cpp:142-505 (net
builders) and 2483-2651 (test_cpu_backend_*), each evaluated single and as a
batch of two, as the reference does.
"""

import numpy as np
import pytest

import kat_nets
import oracle


@pytest.mark.parametrize("name", sorted(kat_nets.ALL))
def test_reference_kat(name):
    fmt, tensors, planes, expect = kat_nets.ALL[name]()
    net = oracle.OracleNet(fmt, tensors)
    single = net.evaluate_batch(planes[None])
    batch = net.evaluate_batch(np.stack([planes, planes]))
    tol = expect["tol"]
    for out in (single, batch):
        last = out["policy"].shape[0] - 1
        for idx, want in expect.get("policy", {}).items():
            assert abs(out["policy"][last, idx] - want) < tol, (idx, out["policy"][last, idx])
        for idx, (lo, hi) in expect.get("policy_range", {}).items():
            assert lo < out["policy"][last, idx] < hi
        assert abs(out["value"][last] - expect["value"]) < tol
    # Batched rows are independent: both rows identical.
    assert np.array_equal(batch["policy"][0], batch["policy"][1])


def test_promotion_logit_quirk_pins_index_1793():
    """policy[1793] (a7a8r) = 15 fixes the reference's mixed 3x64 / 8x8x3
    promotion indexing (cpu_network.cpp:959-1001): its QK term reads pair
    p % 64 = 1 (Q[48].K[57] = 0) and its offset term K[56].(ppo[1] + ppo[3])
    = 5 * 3; reading the QK term in 8x8x3 order (Q[48].K[56] = 10) would give
    25.  policy[1792] (a7a8q) = Q[48].K[56] + K[56].ppo[0] = 10 + 5."""
    fmt, tensors, planes, _ = kat_nets.attention_policy_map()
    out = oracle.OracleNet(fmt, tensors).evaluate_batch(planes[None])
    assert out["policy"][0, 1793] == pytest.approx(15.0, abs=1e-6)
    assert out["policy"][0, 1792] == pytest.approx(15.0, abs=1e-6)
