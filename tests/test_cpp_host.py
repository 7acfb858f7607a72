"""Runs the C++ test programs built by `make -C vllm-cpp_amd` (tests/cpp/*.cpp)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "vllm-cpp_amd", "_build")


def _run(name, timeout):
    exe = os.path.join(BUILD, name)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} not built: run __graft_entry__.build() or make -C vllm-cpp_amd")
    r = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout


def test_block_manager_cpp():
    """The reference's BlockManager unit assertions, restated (CPU only)."""
    _run("test_block_manager", 60)


@pytest.mark.gpu
def test_host_api_gpu():
    """KVCache / paged_attention_forward through the C++ API on the GPU."""
    _run("test_host_gpu", 120)


@pytest.mark.gpu
def test_attention_step_gpu():
    """AttentionMetadata + PagedAttentionLayer (batched RoPE + append + attention of a
    whole step) against the oracle's per-token restatement of the reference."""
    _run("test_attention_step", 120)
