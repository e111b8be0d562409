"""Check order of the sdpa front, ported from the reference's tests/test_sdpa_shapes.py:59-119."""

from __future__ import annotations

from types import ModuleType

import pytest

from tests.fakes import FakeTensor, make_torch_module
from tiledattention._errors import (
    DTypeNotSupportedError,
    InvalidShapeError,
    UnsupportedPlatformError,
)
from tiledattention._runtime import _reset_runtime_cache_for_tests
from tiledattention.sdpa import sdpa


def _patch_runtime_dependency_modules(monkeypatch: pytest.MonkeyPatch) -> None:
    import tiledattention._runtime as runtime

    monkeypatch.setattr(runtime, "_get_native_library", lambda: ModuleType("libtiledattn"))


def _gpu_torch(monkeypatch):
    import tiledattention._runtime as runtime

    torch_mod = make_torch_module(cuda_available=True)
    monkeypatch.setattr(runtime, "_get_torch_module", lambda: torch_mod)
    _patch_runtime_dependency_modules(monkeypatch)
    return torch_mod


def test_sdpa_prefers_runtime_error_on_cpu_path(monkeypatch: pytest.MonkeyPatch) -> None:
    import tiledattention._runtime as runtime

    monkeypatch.setattr(runtime, "_get_torch_module", lambda: make_torch_module(cuda_available=False))
    _reset_runtime_cache_for_tests()
    with pytest.raises(UnsupportedPlatformError):
        sdpa(None, None, None)


def test_sdpa_validates_rank(monkeypatch: pytest.MonkeyPatch) -> None:
    torch_mod = _gpu_torch(monkeypatch)
    q = FakeTensor(shape=(1, 2, 64), dtype=torch_mod.float16, device="cuda:0", is_cuda=True)
    _reset_runtime_cache_for_tests()
    with pytest.raises(InvalidShapeError, match=r"\[B, H, S, D\]"):
        sdpa(q, q, q)


def test_sdpa_validates_dtype(monkeypatch: pytest.MonkeyPatch) -> None:
    _gpu_torch(monkeypatch)
    q = FakeTensor(shape=(1, 2, 64, 64), dtype=object(), device="cuda:0", is_cuda=True)
    _reset_runtime_cache_for_tests()
    with pytest.raises(DTypeNotSupportedError, match="float16"):
        sdpa(q, q, q)


def test_sdpa_valid_input_reaches_kernel_stub(monkeypatch: pytest.MonkeyPatch) -> None:
    import tiledattention.sdpa as sdpa_mod

    torch_mod = _gpu_torch(monkeypatch)
    seen = {}

    def fake_run(q, k, v, *, causal, scale):
        seen.update(causal=causal, scale=scale)
        return "ok"

    monkeypatch.setattr(sdpa_mod, "run_flash_fwd", fake_run)
    q = FakeTensor(shape=(1, 2, 64, 64), dtype=torch_mod.float16, device="cuda:0", is_cuda=True)
    _reset_runtime_cache_for_tests()
    assert sdpa(q, q, q) == "ok"
    assert seen == {"causal": False, "scale": 0.125}


# ---- further order and message checks restated from sdpa.py:37-48 and checks.py:24-55 ----

@pytest.mark.parametrize("causal", [1, "yes", None])
def test_causal_must_be_bool_before_runtime_gate(monkeypatch, causal) -> None:
    import tiledattention._runtime as runtime

    monkeypatch.setattr(runtime, "_get_torch_module", lambda: make_torch_module(cuda_available=False))
    _reset_runtime_cache_for_tests()
    with pytest.raises(InvalidShapeError, match="causal must be a bool"):
        sdpa(None, None, None, causal=causal)


@pytest.mark.parametrize("scale", [0, -1.0, "0.5", complex(1, 0)])
def test_scale_must_be_positive_real(monkeypatch, scale) -> None:
    import tiledattention._runtime as runtime

    monkeypatch.setattr(runtime, "_get_torch_module", lambda: make_torch_module(cuda_available=False))
    _reset_runtime_cache_for_tests()
    with pytest.raises(InvalidShapeError, match="scale must be a positive number"):
        sdpa(None, None, None, scale=scale)


def test_scale_true_passes_as_one(monkeypatch) -> None:
    import tiledattention.sdpa as sdpa_mod

    torch_mod = _gpu_torch(monkeypatch)
    got = []
    monkeypatch.setattr(sdpa_mod, "run_flash_fwd", lambda *a, **kw: got.append(kw["scale"]) or "ok")
    q = FakeTensor(shape=(1, 1, 8, 64), dtype=torch_mod.float16, device="cuda:0", is_cuda=True)
    _reset_runtime_cache_for_tests()
    sdpa(q, q, q, scale=True)
    assert got == [1.0]


def test_zero_head_dim_default_scale_raises(monkeypatch) -> None:
    import tiledattention.sdpa as sdpa_mod

    torch_mod = _gpu_torch(monkeypatch)
    monkeypatch.setattr(sdpa_mod, "run_flash_fwd", lambda *a, **kw: "ok")
    q = FakeTensor(shape=(1, 1, 8, 0), dtype=torch_mod.float16, device="cuda:0", is_cuda=True)
    _reset_runtime_cache_for_tests()
    with pytest.raises(ZeroDivisionError):
        sdpa(q, q, q)


def test_validation_order_and_messages(monkeypatch) -> None:
    torch_mod = _gpu_torch(monkeypatch)
    f16, bf16 = torch_mod.float16, torch_mod.bfloat16
    good = FakeTensor(shape=(1, 2, 16, 64), dtype=f16, device="cuda:0", is_cuda=True)
    _reset_runtime_cache_for_tests()
    with pytest.raises(InvalidShapeError, match="k must be a torch.Tensor"):
        sdpa(good, None, good)
    cpu = FakeTensor(shape=(1, 2, 16, 64), dtype=f16, device="cpu", is_cuda=False)
    with pytest.raises(InvalidShapeError, match="v must be a CUDA tensor"):
        sdpa(good, good, cpu)
    other = FakeTensor(shape=(1, 2, 32, 64), dtype=f16, device="cuda:0", is_cuda=True)
    with pytest.raises(InvalidShapeError, match="matching shape"):
        sdpa(good, other, good)
    dev1 = FakeTensor(shape=(1, 2, 16, 64), dtype=f16, device="cuda:1", is_cuda=True)
    with pytest.raises(InvalidShapeError, match="same CUDA device"):
        sdpa(good, dev1, good)
    mixed = FakeTensor(shape=(1, 2, 16, 64), dtype=bf16, device="cuda:0", is_cuda=True)
    with pytest.raises(DTypeNotSupportedError, match="identical dtype"):
        sdpa(good, mixed, good)
    # rank is checked per tensor before the device check of the same tensor
    bad_rank_cpu = FakeTensor(shape=(2, 16, 64), dtype=f16, device="cpu", is_cuda=False)
    with pytest.raises(InvalidShapeError, match=r"\[B, H, S, D\]"):
        sdpa(good, bad_rank_cpu, good)
