"""The reference's example.py flow through a kernel package laid out by
tiledattention_amd.kernel_build: load ``build/<variant>/tiledattention`` by the local
loader's rule and run its ``sdpa`` on the C1 workload (example.py:19-24)."""
from __future__ import annotations

import importlib

import pytest

from tests.parity_util import as_f32, check_close, inputs, oracle_f32, say

pytestmark = pytest.mark.gpu


def test_example_flow_through_the_local_kernel_package(gpu, tmp_path):
    import torch

    kb = importlib.import_module("tiledattention_amd.kernel_build")
    pkg = kb.write_kernel_package(tmp_path / "build")
    kernel = kb.load_local_kernel(tmp_path)
    q, k, v = inputs((1, 2, 64, 64), "float16", 0)
    dev = torch.device("cuda")
    say("kernel package: example.py workload (1,2,64,64) fp16 causal through the local kernel")
    out = kernel.sdpa(q.to(dev), k.to(dev), v.to(dev), causal=True)
    torch.cuda.synchronize()
    assert out.shape == (1, 2, 64, 64) and out.dtype == torch.float16
    check_close(as_f32(out), oracle_f32(q, k, v, causal=True), "float16", what="local kernel package C1")
    native = importlib.import_module(f"{kernel.__name__}._lib")
    assert native._lib is not None and str(pkg / "lib") in native._lib._name
