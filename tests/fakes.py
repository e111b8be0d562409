"""Fake torch modules for CPU tests of the runtime gate and the sdpa front.

Same idea as the reference's tests (tests/test_errors.py:11-28, tests/test_sdpa_shapes.py:17-49):
a ``ModuleType`` named torch with just the attributes the gate reads, re-targeted to what
the ROCm gate checks (``version.hip``, ``cuda.get_device_properties(i).gcnArchName``).
"""

from __future__ import annotations

from dataclasses import dataclass
from types import ModuleType, SimpleNamespace


@dataclass
class FakeTensor:
    shape: tuple[int, ...]
    dtype: object
    device: str
    is_cuda: bool

    @property
    def ndim(self) -> int:
        return len(self.shape)


def make_torch_module(*, cuda_available: bool, arch: str = "gfx950:sramecc+:xnack-",
                      hip: str | None = "7.0") -> ModuleType:
    torch_mod = ModuleType("torch")
    torch_mod.Tensor = FakeTensor
    torch_mod.float16 = object()
    torch_mod.bfloat16 = object()
    torch_mod.version = SimpleNamespace(hip=hip)

    class FakeCuda:
        @staticmethod
        def is_available() -> bool:
            return cuda_available

        @staticmethod
        def current_device() -> int:
            return 0

        @staticmethod
        def get_device_properties(_device_index: int):
            return SimpleNamespace(gcnArchName=arch)

    torch_mod.cuda = FakeCuda()
    return torch_mod
