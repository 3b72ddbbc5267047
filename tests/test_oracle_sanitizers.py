"""The oracle under sanitizers (CPU): oracle/sanitize.sh builds refcpu.c with
AddressSanitizer + UndefinedBehaviorSanitizer and with ThreadSanitizer and
runs the oracle's own tests (test_oracle.py, test_golden.py) against each
build; any report fails the run."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _runtime(name: str) -> bool:
    gcc = shutil.which("gcc")
    if not gcc:
        return False
    p = subprocess.run([gcc, f"-print-file-name={name}"], capture_output=True, text=True)
    return p.returncode == 0 and Path(p.stdout.strip()).is_absolute()


@pytest.mark.skipif(not (_runtime("libasan.so") and _runtime("libtsan.so")),
                    reason="gcc sanitizer runtimes not installed")
def test_oracle_clean_under_asan_ubsan_and_tsan():
    p = subprocess.run(["bash", str(ROOT / "oracle" / "sanitize.sh")], capture_output=True,
                       text=True, timeout=600)
    assert p.returncode == 0, p.stdout[-4000:] + p.stderr[-4000:]
    assert "sanitizers: clean" in p.stdout
    summaries = [ln for ln in p.stdout.splitlines() if " passed" in ln]
    assert len(summaries) == 2 and not any("failed" in ln or "error" in ln for ln in summaries)
