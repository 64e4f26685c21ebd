"""The C++ host API (aurora_amd/csrc/aurora.hpp: GpuContext, GpuBuffer<T>,
the kernel structs, DecoderTransformerGpu, KvCacheGpu) compiled with g++ and
linked against libaurora_hip.so (tests/cpp/api_check.cpp)."""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "tests" / "cpp" / "api_check.cpp"
BIN = ROOT / "tests" / "cpp" / "api_check"


def compile_api_check(out: Path) -> None:
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-o", str(out), str(SRC), f"-I{ROOT / 'include'}",
           f"-L{ROOT / 'aurora_amd'}", "-laurora_hip", f"-Wl,-rpath,{ROOT / 'aurora_amd'}",
           "-Wl,-rpath,$ORIGIN/../../aurora_amd", "-Wl,-rpath,/opt/rocm/lib"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)


def test_cpp_api_builds_and_fails_cleanly_without_gpu(tmp_path):
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU host: the gpu-marked test runs the API")
    exe = tmp_path / "api_check"
    compile_api_check(exe)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "OK no-gpu" in res.stdout


@pytest.mark.gpu
def test_cpp_api_on_gpu():
    assert BIN.exists(), f"{BIN} is missing: __graft_entry__.build() compiles it"
    res = subprocess.run([str(BIN), "gpu"], capture_output=True, text=True, timeout=120)
    print(res.stdout, flush=True)
    assert res.returncode == 0 and "OK gpu" in res.stdout, res.stdout + res.stderr
