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


def test_gguf_info(tmp_path):
    """gguf-info reads a file's table without a GPU."""
    from gguf_models import build_gguf
    p = str(tmp_path / "m.gguf")
    build_gguf(p, L=2, hidden=512, ffn=256, E=8, n_sel=2, shared=(1,), vocab=300)
    r = run("gguf-info", p)
    assert r.returncode == 0
    assert "GGUF v3" in r.stdout and "qwen3moe" in r.stdout and "15 tensors" in r.stdout
    assert "blk.1.ffn_down_shexp.weight" in r.stdout and "type 14 dims 256 512 8  860160 bytes" in r.stdout
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUF\x63\0\0\0")
    r = run("gguf-info", str(bad))
    assert r.returncode == 1 and "GGUF version 99" in r.stdout


@pytest.mark.gpu
def test_gguf_check(tmp_path):
    """gguf-check runs every MoE layer of a file, routed by its own router."""
    from gguf_models import build_gguf
    p = str(tmp_path / "m.gguf")
    build_gguf(p, L=2, hidden=1024, ffn=512, E=16, n_sel=4, shared=(1,), vocab=300)
    r = run("gguf-check", p)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("PASS") == 2 and "+ shared" in r.stdout and "2 MoE layer(s), 0 failed" in r.stdout
