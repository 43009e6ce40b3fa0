"""A seeded mutation harness over the three parsers that take untrusted
bytes (the roles of the reference's test/fuzz/binary_formats.cc): the plan
loader + validator, the .sds reader and the checkpoint reader. The backend's
host-only sources are built with AddressSanitizer and UBSan into
tests/fuzz/fuzz_formats.cc's driver (g++, no GPU code); mutated seeds must
never crash, over-read or overflow, and every rejection must be one
"<unit>: <message>" line naming the parser's unit. Host only."""
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

from helpers import compile_workload
from seeml_amd import _lib, feeder

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "see-ml_amd", "csrc")


@pytest.fixture(scope="module")
def driver():
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    d = tempfile.mkdtemp(prefix="seeml_fuzz_")
    exe = os.path.join(d, "fuzz_formats")
    cmd = ["g++", "-std=c++20", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-pthread",
           os.path.join(ROOT, "tests", "fuzz", "fuzz_formats.cc"),
           os.path.join(CSRC, "plan_checks.cc"), os.path.join(CSRC, "feeder.cc"),
           os.path.join(CSRC, "checkpoint.cc"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    yield exe, d
    shutil.rmtree(d, ignore_errors=True)


def _seeds(d):
    for name in ("f1", "q1", "k2", "c3s"):
        _, p = compile_workload(name)
        open(os.path.join(d, f"{name}.seeu"), "wb").write(bytes(p.blob))
    x = np.arange(12 * 5, dtype=np.float32)
    feeder.Dataset.from_memory(x, np.arange(12, dtype=np.int32).tobytes(), 12, 5, 1).save(
        os.path.join(d, "rows.sds"))
    feeder.Dataset.from_memory(x, (x[:24] * 0.5).astype(np.float32).tobytes(), 12, 5, 2,
                               label_dim=2).save(os.path.join(d, "dense.sds"))
    feeder.Dataset.from_tokens(np.arange(4 * 9, dtype=np.int32) % 7, 4, 8).save(
        os.path.join(d, "tokens.sds"))
    import ctypes as C
    payload = np.random.default_rng(1).standard_normal(300).astype(np.float32).tobytes()
    buf = (C.c_uint8 * len(payload)).from_buffer_copy(payload)
    err = C.create_string_buffer(256)
    path = os.path.join(d, f"{0xabc123:x}_{len(payload)}.sekp")
    assert _lib.lib().seeml_hip_checkpoint_write(path.encode(), 0xabc123, 5, buf, len(payload),
                                                 err, 256) == 0


@pytest.mark.parametrize("rng_seed", [1, 2])
def test_mutated_inputs_never_crash_and_reject_with_a_unit(driver, rng_seed):
    exe, d = driver
    seeds = os.path.join(d, f"seeds{rng_seed}")
    os.makedirs(seeds, exist_ok=True)
    _seeds(seeds)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, seeds, "700", str(rng_seed)], capture_output=True, text=True,
                       env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    nums = [int(t) for t in r.stdout.replace("|", " ").split() if t.isdigit()]
    plans_rej, plans_acc, sds_rej, sds_acc, ck_rej, ck_acc = nums
    assert plans_rej > 100 and sds_rej > 100 and ck_rej > 100, r.stdout
    assert plans_acc > 0 and sds_acc > 0, r.stdout  # some mutants survive and are exercised
