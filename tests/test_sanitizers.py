"""Host code under sanitizers (CPU only, no GPU needed).

* The C++ ``HipNetwork`` adapter over a CPU fake of the C ABI
  (``tests/native/mfh_fake.cpp``), built with ThreadSanitizer: eight threads
  call EvaluateBatch / EvaluateBatchPriors / Evaluate on one net at once
  (MCTS workers, reference src/mcts/search.cpp:433) and must get their
  serial results bit for bit with no race reported; injected failures and
  non-finite outputs drive the retry-once-then-throw path (reference
  src/nn/cuda/cuda_network.cpp:199-231, 444-458).
* The network-file reader (``weights_file.cpp``) built with AddressSanitizer
  and UndefinedBehaviorSanitizer, on every fixture, every prefix of each
  fixture (``truncated.pb`` among them) and seeded byte-level mutations.
"""

import glob
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NATIVE = os.path.join(ROOT, "tests", "native")
HOST = os.path.join(ROOT, "metalfish_amd", "csrc", "host")
NETFILES = os.path.join(ROOT, "tests", "golden", "netfiles")


def _gxx():
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not available")
    return gxx


def _build(out, sources, sanitize, libs=()):
    cmd = [_gxx(), "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           f"-fsanitize={sanitize}", "-fno-sanitize-recover=all",
           "-I" + os.path.join(ROOT, "include"), "-I" + HOST, *sources, "-o", out, *libs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr


def test_adapter_concurrent_callers_and_retry_under_tsan(tmp_path):
    exe = str(tmp_path / "adapter_tsan")
    _build(exe, [os.path.join(NATIVE, "adapter_concurrency_test.cpp"),
                 os.path.join(NATIVE, "mfh_fake.cpp"),
                 os.path.join(HOST, "hip_network.cpp")], "thread", ["-lpthread"])
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66")
    proc = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "ThreadSanitizer" not in proc.stderr, proc.stderr
    assert "adapter concurrency ok" in proc.stdout


def test_network_file_reader_under_asan_ubsan(tmp_path):
    exe = str(tmp_path / "netfile_asan")
    _build(exe, [os.path.join(NATIVE, "netfile_fuzz_test.cpp"),
                 os.path.join(HOST, "weights_file.cpp")], "address,undefined", ["-lz"])
    files = sorted(glob.glob(os.path.join(NETFILES, "*.pb")) +
                   glob.glob(os.path.join(NETFILES, "*.pb.gz")))
    assert any(f.endswith("truncated.pb") for f in files)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:allocator_may_return_null=1",
               UBSAN_OPTIONS="print_stacktrace=1")
    proc = subprocess.run([exe, *files], capture_output=True, text=True, env=env, timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "ERROR: AddressSanitizer" not in proc.stderr
    assert "runtime error" not in proc.stderr, proc.stderr
    assert f"{len(files)} files" in proc.stdout
