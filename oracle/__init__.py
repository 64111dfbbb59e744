"""CPU ORACLE -- TEST INFRASTRUCTURE ONLY.

A restatement of MetalFish's reference CPU transformer backend
(``src/nn/cpu/cpu_network.cpp``): ``plan.py`` resolves the step list and data
flow, ``cpu_ref.c`` executes it with the reference's fp32 loop order.  Only
tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may use
it, as the checker; the product path (``metalfish_amd``) never imports it.

Every function is pinned by a reference golden vector, a reference KAT or a
closed-form / brute-force check (listed in ``plan.py``'s docstring).  No part
is "parity unpinned".
"""

from __future__ import annotations

import concurrent.futures as _futures
import os

import numpy as np

from . import _lib
from .plan import NetFormat, ResolvedProgram  # noqa: F401
from .policy_tables import gather_table


def pack_planes(planes):
    """PackInputPlanesRaw (reference src/nn/input_plane_packing.h:61-83)."""
    planes = np.ascontiguousarray(planes, dtype=np.float32).reshape(-1, 112, 64)
    b = planes.shape[0]
    masks = np.zeros((b, 112), dtype=np.uint64)
    values = np.zeros((b, 112), dtype=np.float32)
    if b:
        _lib.lib().or_pack_planes(planes.ctypes.data, b, masks.ctypes.data, values.ctypes.data)
    return masks, values


class OracleNet:
    """CPU reference network for one weights set."""

    def __init__(self, fmt: NetFormat, tensors: dict, policy_head="vanilla",
                 value_head="winner"):
        self.fmt = fmt
        self.program = ResolvedProgram(fmt, tensors, policy_head, value_head,
                                       gather=gather_table())

    def _run_chunk(self, masks, values):
        p = self.program
        b = masks.shape[0]
        policy = np.zeros((b, p.policy_width), dtype=np.float32)
        value = np.zeros((b, p.value_width), dtype=np.float32)
        moves = np.zeros((b,), dtype=np.float32)
        masks = np.ascontiguousarray(masks, dtype=np.uint64)
        values = np.ascontiguousarray(values, dtype=np.float32)
        rc = _lib.lib().or_run(b, masks.ctypes.data, values.ctypes.data,
                               ctypes_addr(p.c_steps), len(p.records), p.n_buffers,
                               p.policy_buf, policy.ctypes.data, p.policy_width,
                               p.value_buf, value.ctypes.data, p.value_width,
                               p.moves_buf, moves.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"oracle step execution failed (code {rc})")
        return policy, value, moves

    def run_packed(self, masks, values, threads=None):
        """Raw outputs for packed inputs; positions are independent, so the
        batch is split across threads without changing any result bit."""
        masks = np.asarray(masks).reshape(-1, 112)
        values = np.asarray(values).reshape(-1, 112)
        b = masks.shape[0]
        if b == 0:
            return (np.zeros((0, 1858), np.float32),
                    np.zeros((0, self.program.value_width), np.float32),
                    np.zeros((0,), np.float32))
        threads = threads or min(b, os.cpu_count() or 1)
        chunks = np.array_split(np.arange(b), min(threads, b))
        with _futures.ThreadPoolExecutor(len(chunks)) as ex:
            parts = list(ex.map(lambda c: self._run_chunk(masks[c], values[c]), chunks))
        return tuple(np.concatenate([p[i] for p in parts]) for i in range(3))

    def evaluate_batch(self, planes, threads=None):
        """NetworkOutput fields for float planes [B,112,64]."""
        masks, values = pack_planes(planes)
        policy, raw_value, moves = self.run_packed(masks, values, threads)
        out = {"policy": policy}
        if self.fmt.wdl:
            out["wdl"] = raw_value
            out["value"] = raw_value[:, 0] - raw_value[:, 2]
        else:
            out["wdl"] = np.zeros((policy.shape[0], 3), np.float32)
            out["value"] = raw_value[:, 0]
        if self.fmt.moves_left:
            out["moves_left"] = moves
        return out


def ctypes_addr(arr):
    import ctypes
    return ctypes.addressof(arr)


def fast_exp(x):
    """FastMath::FastExp (reference src/mcts/core.h:38-44), elementwise on
    float32: clamp to [-88, 88] with std::min/std::max comparisons (NaN ->
    88), then the binary32 pattern int(x * 12102203) + 1065353216
    (Schraudolph's method)."""
    x = np.asarray(x, dtype=np.float32)
    x = np.where(x < np.float32(88.0), x, np.float32(88.0)).astype(np.float32)
    x = np.where(np.float32(-88.0) < x, x, np.float32(-88.0)).astype(np.float32)
    prod = (x * np.float32(12102203.0)).astype(np.float32)
    bits = np.trunc(prod).astype(np.int64) + 1065353216
    return bits.astype(np.int32).view(np.float32)


def mcts_priors(logits, indices, softmax_temp):
    """Priors of one position's legal moves as the reference's MCTS forms
    them: BuildResult's gather (src/mcts/evaluator.cpp:193-204: logit 0 for an
    index outside the policy) and ApplyNNPolicyToNode
    (src/mcts/search.cpp:127-199: max, FastExp((l - max) * (1 / temp)),
    sequential float32 sum, multiply by 1 / sum, or 1 / n when the sum is not
    positive).  ``logits`` [1858] float32, ``indices`` the move list."""
    logits = np.asarray(logits, dtype=np.float32)
    idx = np.asarray(indices, dtype=np.int64)
    n = idx.size
    if n == 0:
        return np.zeros(0, np.float32)
    ok = (idx >= 0) & (idx < logits.size)
    l = np.where(ok, logits[np.where(ok, idx, 0)], np.float32(0.0)).astype(np.float32)
    m = np.float32(-np.inf)
    for v in l:  # the reference's sequential "if (l > max) max = l"
        if v > m:
            m = v
    inv_temp = np.float32(1.0) / np.float32(softmax_temp)
    p = fast_exp(((l - m).astype(np.float32) * inv_temp).astype(np.float32))
    total = np.add.accumulate(p, dtype=np.float32)[-1]
    if not total > np.float32(0.0) and not np.isnan(total):
        return np.full(n, np.float32(1.0) / np.float32(n), dtype=np.float32)
    inv = np.float32(1.0) / total
    return (p * inv).astype(np.float32)
