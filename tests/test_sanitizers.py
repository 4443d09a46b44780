"""The block manager and the C ABI's host paths under AddressSanitizer and
ThreadSanitizer (krill_amd/csrc/sanitize.sh): the host-only-pool tests,
including the 8-thread hammer, run against instrumented copies of the
library.  CPU only; needs the kernel objects of a normal build."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "krill_amd", "csrc")
CLANG = "/opt/rocm/llvm/bin/clang++"


@pytest.mark.skipif(not os.path.exists(CLANG), reason="ROCm clang++ not present")
@pytest.mark.skipif(not os.path.exists(os.path.join(CSRC, "_build", "attn_mfma.o")),
                    reason="library objects not built (run the Makefile first)")
def test_host_code_is_clean_under_asan_and_tsan():
    r = subprocess.run([os.path.join(CSRC, "sanitize.sh")], capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert tail.count("passed") == 2 and "failed" not in tail, tail
