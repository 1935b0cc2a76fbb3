"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

The GGUF loader, tokenizer and C-ABI argument checks read untrusted files and
caller buffers.  This test builds libtinyengine_san.so (their host code
compiled with -fsanitize=address,undefined, no recovery; see
tinymetalagent_amd/build.py build_sanitized) and runs the loader / tokenizer
tests (including the corrupted-file fuzz) and the ABI guard tests against it
in a child process with the clang ASan runtime preloaded.  Any sanitizer
report aborts the child, so a non-zero exit or a report in its output fails.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_loader_tokenizer_abi_clean_under_asan_ubsan():
    if shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").is_file():
        pytest.skip("hipcc not available")
    sys.path.insert(0, str(ROOT))
    from tinymetalagent_amd import build as B

    if not all((B.BUILD / (Path(s).stem + ".o")).is_file() for s in B.HIP_SOURCES):
        pytest.skip("normal build objects missing (run __graft_entry__.build() first)")
    lib = B.build_sanitized()
    env = dict(os.environ)
    env.update(LD_PRELOAD=str(B.asan_runtime()), ASAN_OPTIONS="detect_leaks=0",
               UBSAN_OPTIONS="print_stacktrace=1", TINYENGINE_LIBRARY=str(lib))
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
           str(ROOT / "tests" / "test_model_cpu.py"), str(ROOT / "tests" / "test_abi.py")]
    proc = subprocess.run(cmd, cwd=str(ROOT), env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=900)
    out = proc.stdout
    print(out[-3000:])
    assert proc.returncode == 0, out[-3000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out
    assert " passed" in out
