"""The attention planner (fast_v2_amd/csrc/attn_plan.h: kernel family, workspace sizes,
launch grids, call validation) built for the host with AddressSanitizer and
UndefinedBehaviorSanitizer and swept over 3.3 M descriptors whose fields run out to
their limits (batch to 2^31 - 1, lengths to 2^31 - 1, page counts, kv_split up to 2^30,
up to 65535 KV heads). Any sanitizer report aborts the sweep; the sweep's own checks
(exact 128-bit workspace sizes, grids within launch limits and covering the work, each
kernel family's preconditions, refusals carrying an error message) must all pass.
CPU only: g++ on the header alone, no HIP."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
@pytest.mark.parametrize("defines", [[], ["-DFDLLM_DECODE_TEAMS=1"]], ids=["default", "decode_one_team"])
def test_planner_sweep_under_asan_ubsan(tmp_path, defines):
    """Swept for the default build and for the build option of one team per split decode
    workgroup (twice the slots per KV head)."""
    exe = tmp_path / "plan_sweep"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", *defines,
           "-I", str(ROOT / "include"), "-I", str(ROOT / "fast_v2_amd" / "csrc"),
           str(ROOT / "tests" / "plan_sweep.cc"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=300)
    # verify_asan_link_order=0: the sanitizer runtime need not come first among the
    # libraries the environment preloads
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    words = r.stdout.split()
    tried, accepted = int(words[1]), int(words[3])
    kinds = [int(x) for x in words[5:12]]
    assert tried == 3326400 and accepted > 0
    # the sweep reaches every kernel family
    assert all(k > 0 for k in kinds), kinds
