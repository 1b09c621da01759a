"""The host parsers that read untrusted files (weight packs, their JSON
manifest, the model config) under AddressSanitizer and
UndefinedBehaviorSanitizer: tests/host/parsers_fuzz.cpp checks a valid pack
reads back exactly, that hand-picked malformed packs are rejected, and that
thousands of deterministic mutants either load in bounds or throw. The
reference runs its suites under compute-sanitizer (tests/run_sanitizers.sh);
GPU sanitizers are not available on the target pool, so host code is what
runs sanitized here."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_pack_and_config_parsers_under_sanitizers(tmp_path):
    exe = tmp_path / "parsers_fuzz"
    flags = ["-fsanitize=address,undefined,float-cast-overflow", "-fno-sanitize-recover=all", "-static-libasan"]
    build = subprocess.run(["g++", "-std=c++17", "-O1", "-g", *flags, "-I", str(ROOT / "opworks_amd/include/runtime"),
                            str(ROOT / "tests/host/parsers_fuzz.cpp"), "-o", str(exe)],
                           capture_output=True, text=True, timeout=300)
    assert build.returncode == 0, build.stderr[-4000:]
    run = subprocess.run([str(exe), str(tmp_path), "6000"], capture_output=True, text=True, timeout=300)
    print(run.stdout)
    assert run.returncode == 0, (run.stdout + run.stderr)[-4000:]
    assert "0 failures" in run.stdout
