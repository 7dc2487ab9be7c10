"""The fused kernel's work partition (detail::ShareMap, innerq_amd/csrc/iq_gemv.h),
checked on the host: every split covered once, run slots distinct and dense per
(batch, KV head).  The partition decides where each run's partial goes and which
slots the combine kernels read, so a gap or a collision would lose or double a
piece of the softmax."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "native", "share_map_check.cpp")
OUT = os.path.join(HERE, "..", "innerq_amd", "_build", "share_map_check")


@pytest.fixture(scope="module")
def checker():
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    subprocess.run([hipcc, "-x", "hip", "--offload-host-only", "-std=c++20", "-O1", SRC, "-o", OUT], check=True,
                   capture_output=True)
    return OUT


def run(checker, cases):
    inp = "".join(f"{g} {h} {s} {e}\n" for g, h, s, e in cases)
    r = subprocess.run([checker], input=inp, capture_output=True, text=True, check=True)
    lines = r.stdout.split("\n")[:-1]
    assert len(lines) == len(cases)
    return lines


def test_share_map_invariants(checker):
    cases = []
    for grid in (1, 7, 8, 16, 24, 64, 200, 256, 512):
        for nhead in (1, 2, 3, 8, 13, 64, 128, 640):
            for nsplit in (1, 2, 3, 4, 5, 31, 64, 127, 128, 1023):
                # the launches never use more workgroups than splits
                if grid <= nhead * nsplit <= 200000:
                    for e0num in (0, 1, 64, 68, 127):
                        cases.append((grid, nhead, nsplit, e0num))
    lines = run(checker, cases)
    bad = [(c, l) for c, l in zip(cases, lines) if not l.startswith("ok")]
    assert not bad, bad[:5]


def test_share_map_paired_at_benchmark_shapes(checker):
    # headline (64 heads x 128 splits) and a 4-bit config-3 shape (128 x 64):
    # paired on a 256-workgroup grid when asked; config 1 (8 x 32), one split
    # per head, or no pairing asked: plain
    lines = run(checker, [(256, 64, 128, 68), (256, 128, 64, 68), (256, 8, 32, 68), (256, 64, 1, 68),
                          (256, 64, 128, 0)])
    assert lines == ["ok 1", "ok 1", "ok 0", "ok 0", "ok 0"]

