"""The allocator's reuse policy (tl_amd/csrc/block_cache.h) on the CPU: which freed block may
serve which stream's request.  Builds tests/block_cache_test.cpp with g++ and runs it."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_block_cache_policy(tmp_path):
    exe = str(tmp_path / "block_cache_test")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-fsanitize=address,undefined",
                    os.path.join(HERE, "block_cache_test.cpp"), "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
