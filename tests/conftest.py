import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def pytest_collection_modifyitems(config, items):
    # GPU tests fail loudly (no CPU fallback); without a device they are
    # deselected only when the run asked for "not gpu".
    pass


@pytest.fixture(scope="session")
def bt4_bench_oracle():
    """get(fp8=False) -> (weights, planes, legal, oracle outputs) for the
    bench's 256 positions on the BT4-shape net of seed 0, with bf16 or e4m3
    (dequantised) weights; each computed once per session on up to 16 host
    cores, shared by the GPU test modules that hold the bench's
    configurations to the gates."""
    import time

    import oracle
    from metalfish_amd import synth

    cache = {}

    def get(fp8=False):
        if fp8 not in cache:
            spec = synth.SPECS["bt4"]
            weights = synth.make_weights(spec, seed=0, fp8=fp8)
            planes, legal = synth.playout_positions(256, seed=0)
            threads = min(16, os.cpu_count() or 1)
            t0 = time.time()
            ref = oracle.OracleNet(oracle.NetFormat(body_heads=spec.heads),
                                   weights).evaluate_batch(planes, threads=threads)
            print(f"oracle: 256 BT4 positions ({'e4m3' if fp8 else 'bf16'} weights) on "
                  f"{threads} threads in {time.time() - t0:.1f} s", flush=True)
            cache[fp8] = (weights, planes, legal, ref)
        return cache[fp8]

    return get
