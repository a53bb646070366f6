"""The C host logic above the sampler ABI, on the CPU (no GPU, no HIP):

- INTEGRATION.md's drop-in snippet, extracted from the document as it
  stands, compiles as a C11 translation unit against the headers with
  -Wall -Wextra -Werror;
- that snippet and pgl_generate (pumice_amd/csrc/pss_generate.c) run against
  a host stand-in of the ABI (tests/c/fake_sampler.c: the O1 oracle behind
  every entry point) under AddressSanitizer and UBSan, and match a direct O1
  chain in tokens, positions, rng and history rings (tests/c/host_main.c)."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C = os.path.join(ROOT, "tests", "c")
INC = ["-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "pumice_amd", "csrc"),
       "-I" + os.path.join(ROOT, "oracle")]

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")


def _snippet(tmp_path):
    out = subprocess.run([sys.executable, os.path.join(C, "extract_snippet.py"),
                          os.path.join(ROOT, "INTEGRATION.md")], capture_output=True, text=True, check=True)
    p = tmp_path / "snippet.c"
    p.write_text(out.stdout)
    return p


def _gcc(args, cwd):
    r = subprocess.run(["gcc", *args], capture_output=True, text=True, cwd=cwd)
    assert r.returncode == 0, " ".join(args) + "\n" + r.stderr


def test_integration_snippet_compiles_as_c11(tmp_path):
    snip = _snippet(tmp_path)
    assert "generatorSetSampling" in snip.read_text()
    _gcc(["-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic", *INC, "-c", str(snip), "-o",
          str(tmp_path / "snippet.o")], tmp_path)


def test_host_logic_under_asan(tmp_path):
    _snippet(tmp_path)
    san = ["-g", "-O1", "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=all"]
    objs = []
    for src, std in [(os.path.join(ROOT, "oracle", "pss_oracle.c"), "gnu11"),
                     (os.path.join(ROOT, "pumice_amd", "csrc", "pss_generate.c"), "c11"),
                     (os.path.join(C, "fake_sampler.c"), "c11"),
                     (os.path.join(C, "host_main.c"), "c11")]:
        obj = str(tmp_path / (os.path.basename(src) + ".o"))
        _gcc([f"-std={std}", "-Wall", "-Wextra", "-ffp-contract=off", "-mfma", *san, *INC,
              "-I" + str(tmp_path), "-c", src, "-o", obj], tmp_path)
        objs.append(obj)
    exe = str(tmp_path / "host_main")
    _gcc([*san, *objs, "-o", exe, "-lm", "-lpthread"], tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "host logic ok" in r.stdout
