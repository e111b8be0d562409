"""The custom operator on the CPU: registration, the fake kernel's output metadata and checks,
and graph capture with fake CUDA tensors (no GPU needed: nothing is executed)."""

from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")

from tiledattention import torch_op  # noqa: E402  (registers the operator)
from tiledattention._errors import DTypeNotSupportedError, InvalidShapeError  # noqa: E402


def _fake_mode():
    from torch._subclasses.fake_tensor import FakeTensorMode

    return FakeTensorMode()


def test_operator_is_registered():
    assert torch_op.OP_NAME == "tiledattention::sdpa_fwd"
    op = torch.ops.tiledattention.sdpa_fwd.default
    names = [a.name for a in op._schema.arguments]
    assert names == ["q", "k", "v", "causal", "scale", "tile_m", "tile_n", "accum"]
    assert str(op._schema.returns[0].type) == "Tensor"


@pytest.mark.parametrize("shape,dtype", [((2, 4, 100, 80), torch.bfloat16), ((1, 1, 7, 256), torch.float16)])
def test_fake_output_metadata(shape, dtype):
    with _fake_mode():
        q = torch.empty(shape, dtype=dtype, device="cuda")
        out = torch.ops.tiledattention.sdpa_fwd(q, q, q, True, None)
        assert out.shape == q.shape and out.dtype == dtype and out.device == q.device
        assert out.is_contiguous()


def test_fake_applies_the_same_checks():
    with _fake_mode():
        q = torch.empty((1, 2, 8, 64), dtype=torch.float16, device="cuda")
        with pytest.raises(DTypeNotSupportedError, match="identical dtype"):
            torch.ops.tiledattention.sdpa_fwd(q, q, q.to(torch.bfloat16), False, None)
        with pytest.raises(InvalidShapeError, match="matching shape"):
            torch.ops.tiledattention.sdpa_fwd(q, q, q[:, :, :4], False, None)
        with pytest.raises(DTypeNotSupportedError, match="float16 or torch.bfloat16"):
            x = q.float()
            torch.ops.tiledattention.sdpa_fwd(x, x, x, False, None)


def test_graph_capture_keeps_the_operator():
    from torch.fx.experimental.proxy_tensor import make_fx

    def fn(q, k, v):
        return torch.ops.tiledattention.sdpa_fwd(q, k, v, True, 0.1) * 2

    with _fake_mode():
        q = torch.empty((1, 2, 64, 64), dtype=torch.float16, device="cuda")
        g = make_fx(fn, tracing_mode="real")(q, q, q)
    targets = [str(n.target) for n in g.graph.nodes if n.op == "call_function"]
    assert targets[0].startswith("tiledattention.sdpa_fwd")


@pytest.mark.parametrize("tm,tn,acc,msg", [
    (64, 0, -1, "both be 0"), (0, 128, -1, "both be 0"), (32, 64, -1, "Unsupported tile"),
    (128, 256, -1, "Unsupported tile"), (0, 0, 2, "accum must be"), (64, 64, -2, "accum must be"),
])
def test_fake_checks_the_tile_and_accum_arguments(tm, tn, acc, msg):
    with _fake_mode():
        q = torch.empty((1, 2, 8, 64), dtype=torch.float16, device="cuda")
        with pytest.raises(ValueError, match=msg):
            torch.ops.tiledattention.sdpa_fwd(q, q, q, False, None, tm, tn, acc)


def test_overrides_map_to_run_flash_fwd_keywords():
    assert torch_op._overrides(0, 0, -1) == {}
    assert torch_op._overrides(64, 128, -1) == {"tile": (64, 128)}
    assert torch_op._overrides(0, 0, 1) == {"accum": "fp16"}
    assert torch_op._overrides(128, 64, 0) == {"tile": (128, 64), "accum": "fp32"}


def test_operator_kernel_is_the_cpp_library():
    """The schema and the GPU kernel are registered by libtiledattn_torch.so (C++), the fake
    (Meta) kernel by this package: libtorch callers reach the operator without Python."""
    dump = torch._C._dispatch_dump("tiledattention::sdpa_fwd")
    lines = {ln.split(":", 1)[0]: ln for ln in dump.splitlines() if ":" in ln}
    assert "torch_ext.cpp" in lines["debug"]
    assert "torch_ext.cpp" in lines["CUDA"]
    assert "torch_ext.cpp" not in lines["Meta"]
    assert torch._C._dispatch_has_kernel_for_dispatch_key("tiledattention::sdpa_fwd", "CUDA")
    assert not torch._C._dispatch_has_kernel_for_dispatch_key("tiledattention::sdpa_fwd", "CPU")
