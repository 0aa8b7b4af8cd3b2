"""The host-side parsers (tokenizer.cpp, safetensors.cpp) under AddressSanitizer and UBSan: a g++
build of the two sources with tests/fuzz/host_fuzz.cpp, run over randomised valid and corrupted
vocabularies and safetensors files.  Host code only (no HIP, no device).  CPU only."""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT


def test_parsers_under_sanitizers(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    src = os.path.join(ROOT, "universal-dictator_amd", "csrc")
    exe = str(tmp_path / "host_fuzz")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-I" + os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "fuzz", "host_fuzz.cpp"), os.path.join(src, "tokenizer.cpp"),
           os.path.join(src, "safetensors.cpp"), "-o", exe]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, "4000"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, env=env,
                       timeout=300)
    assert r.returncode == 0 and "fuzz ok" in r.stdout, r.stdout[-4000:]
    # the random inputs reached the parsers' success paths too, not only their refusals
    counts = [int(x) for x in r.stdout.replace(",", " ").split() if x.isdigit()]
    assert len(counts) >= 4 and min(counts[1:]) > 0, r.stdout
