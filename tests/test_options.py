"""Backend flag, import isolation and dispatch (reference tests/test_import.py:9-68)."""

import os
import subprocess
import sys

import pytest
import torch

import stackkernels_amd
from stackkernels_amd.torch import _dispatch


def test_root_import_does_not_import_torch():
    code = ("import sys, stackkernels_amd; "
            "assert stackkernels_amd.__version__ == '0.1.0'; "
            "assert stackkernels_amd.get_backend() in ('auto','triton','hip','reference'); "
            "assert 'torch' not in sys.modules, 'torch imported by package root'")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    subprocess.run([sys.executable, "-c", code], check=True, cwd=root)


def test_options_configuration():
    original = stackkernels_amd.get_backend()
    try:
        for name in ("reference", "triton", "hip", "auto"):
            stackkernels_amd.set_backend(name)
            assert stackkernels_amd.get_backend() == name
            assert stackkernels_amd.options().backend == name
        stackkernels_amd.options(backend=" REFERENCE ")
        assert stackkernels_amd.get_backend() == "reference"
        with pytest.raises(ValueError, match="Invalid backend"):
            stackkernels_amd.set_backend("cuda_native")
    finally:
        stackkernels_amd.set_backend(original)


def test_env_backend(monkeypatch):
    from stackkernels_amd._options import Options

    monkeypatch.setenv("STACKKERNELS_BACKEND", "reference")
    assert Options().backend == "reference"
    monkeypatch.setenv("STACKKERNELS_BACKEND", "bogus")
    with pytest.raises(ValueError, match="Invalid backend"):
        Options()


def test_dispatch_rules():
    cpu = torch.zeros(1)
    original = stackkernels_amd.get_backend()
    try:
        stackkernels_amd.set_backend("auto")
        assert _dispatch.should_use_hip(cpu) is False
        stackkernels_amd.set_backend("reference")
        assert _dispatch.should_use_triton(cpu) is False
        for forced in ("hip", "triton"):
            stackkernels_amd.set_backend(forced)
            assert _dispatch.should_use_hip(cpu) is True
    finally:
        stackkernels_amd.set_backend(original)


def test_forced_kernel_backend_on_cpu_tensor_fails_loudly():
    from stackkernels_amd.torch import flash_attention, flash_decode

    q = torch.randn(1, 2, 4, 64)
    original = stackkernels_amd.get_backend()
    try:
        stackkernels_amd.set_backend("hip")
        with pytest.raises(RuntimeError, match="ROCm device tensors"):
            flash_attention(q, q, q)
        with pytest.raises(RuntimeError, match="ROCm device tensors"):
            flash_decode(q[:, :, :1], q, q)
    finally:
        stackkernels_amd.set_backend(original)
