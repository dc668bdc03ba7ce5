"""CPU checks of the row schedule: tests/cpp/test_schedule.cpp, compiled from the library's host
sources (varblockspmm_amd/csrc/schedule.cpp, host_format.cpp), on generated and hand-made matrices.
It checks the step records against the block metadata, that both launch orders (RHS 8/16 and
RHS 32/64) are permutations of the block rows on the same XCDs with bounded work per XCD, the
orders within each XCD, determinism, and that matrices whose rows share few block columns are
scheduled in seconds.  It also checks the launchers' host-side panel check at the edges of the B
and C ranges."""

import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")


def test_schedule_program():
    subprocess.run(["make", "-s", "-C", CPP, "test_schedule"], check=True)
    result = subprocess.run([os.path.join(CPP, "test_schedule")], capture_output=True, text=True, timeout=300)
    print(result.stdout)
    assert result.returncode == 0, result.stdout + result.stderr
    assert result.stdout.strip().endswith("ALL OK")
    assert result.stdout.count("\nok ") + result.stdout.startswith("ok ") == 16


def test_validate_fuzz_program():
    """tests/cpp/test_validate_fuzz.cpp under AddressSanitizer and UBSan: 4000 mutated matrices;
    validate accepts or rejects each without reading outside its arrays or overflowing, and
    accepted mutants schedule inside the matrix."""
    subprocess.run(["make", "-s", "-C", CPP, "test_validate_fuzz"], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1")
    result = subprocess.run([os.path.join(CPP, "test_validate_fuzz")], capture_output=True, text=True, timeout=600,
                            env=env)
    print(result.stdout)
    assert result.returncode == 0, result.stdout + result.stderr
    assert result.stdout.strip().endswith("ALL OK")
