"""The katali-hip harness (the reference engine's cuda-info / cuda-check /
cuda-check-moe / cuda-dp4a-selftest / cuda-bench commands, README.md:13,17,
99-102,309-312) built on the engine-side loader."""
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(REPO, "katali-lab_amd", "katali-hip")


def run(*args, timeout=120):
    assert os.path.exists(CLI), "run python katali-lab_amd/build.py"
    print(f"[cli] {' '.join(args)}", flush=True)
    p = subprocess.run([CLI, *args], capture_output=True, text=True, timeout=timeout)
    print(p.stdout + p.stderr)
    return p


def test_usage_without_command():
    p = run()
    assert p.returncode == 2 and "usage" in p.stderr


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_reports_no_gpu():
    p = run("info")
    assert p.returncode == 2 and "no usable GPU" in p.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("cmd", ["info", "dp4a-selftest", "check", "check-moe"])
def test_checks_pass(cmd):
    p = run(cmd)
    assert p.returncode == 0, p.stdout + p.stderr
    if cmd != "info":
        assert "FAIL" not in p.stdout and "PASS" in p.stdout


@pytest.mark.gpu
def test_bench_reports_a_rate():
    p = run("bench", "4")
    assert p.returncode == 0, p.stderr
    assert "GB/s" in p.stdout and "tok/s" in p.stdout
