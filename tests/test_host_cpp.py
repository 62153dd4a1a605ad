"""Runs the C++ host-layer test programs (tests/cpp, built by __graft_entry__.build()): the CPU one
checks argument validation and the inv_freq producer; the GPU one checks RmsNorm / Embedding /
GatedMlp / RoPE modules against the CPU oracle."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "build")


def run(name):
    path = os.path.join(BIN, name)
    assert os.path.exists(path), f"{path} is not built: run __graft_entry__.build()"
    p = subprocess.run([path], capture_output=True, text=True, timeout=120)
    print(p.stdout, p.stderr)
    assert p.returncode == 0, p.stdout + p.stderr


def test_host_layer_cpu():
    run("test_host_cpu")


@pytest.mark.gpu
def test_host_layer_gpu():
    run("test_host_gpu")
