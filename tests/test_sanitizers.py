"""AddressSanitizer + UndefinedBehaviorSanitizer over the CPU code: the oracle
(oracle/momij_oracle.c) and the host-side draft sources (momij_amd/csrc/drafts.cpp), built
with gcc/g++ and driven by tests/sanitize/san_driver.cpp on small seeded inputs and the edge
cases their callers hit.  Any invalid access, leak or undefined operation aborts the driver."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1", "-fopenmp"]


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("g++") is None,
                    reason="gcc/g++ not installed")
def test_oracle_and_drafts_under_asan_ubsan(tmp_path):
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "oracle")]
    objs = []
    o1 = str(tmp_path / "oracle.o")
    subprocess.run(["gcc", "-std=gnu11", "-ffp-contract=off", *SAN, *inc, "-c",
                    os.path.join(ROOT, "oracle", "momij_oracle.c"), "-o", o1], check=True)
    objs.append(o1)
    o2 = str(tmp_path / "drafts.o")
    subprocess.run(["g++", "-std=c++17", *SAN, *inc, "-c",
                    os.path.join(ROOT, "momij_amd", "csrc", "drafts.cpp"), "-o", o2], check=True)
    objs.append(o2)
    exe = str(tmp_path / "san_driver")
    subprocess.run(["g++", "-std=c++17", *SAN, *inc,
                    os.path.join(ROOT, "tests", "sanitize", "san_driver.cpp"), *objs, "-o", exe,
                    "-lm"], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="2")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
    print(r.stdout[-2000:], r.stderr[-4000:])
    assert r.returncode == 0, r.stderr[-4000:]
    assert "all cases ran" in r.stdout
    assert "runtime error" not in r.stderr
