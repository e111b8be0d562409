"""Loader of the committed golden fixtures (numpy .npz, loaded without pickle)."""

from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def load_fixture(name: str) -> dict:
    """Return q/k/v as torch CPU tensors plus the stored oracle outputs and metadata."""
    import torch

    with np.load(HERE / f"{name}.npz", allow_pickle=False) as z:
        data = {key: z[key] for key in z.files}
    dtype = str(data["dtype"])
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    out = {
        "dtype": dtype,
        "causal": bool(data["causal"]),
        "seed": int(data["seed"]),
        "out_f32": data["out_f32"],
        "out_f64": data["out_f64"],
        "q_bits": data["q"],
        "k_bits": data["k"],
        "v_bits": data["v"],
    }
    for key in ("q", "k", "v"):
        out[key] = torch.from_numpy(data[key].view(np.int16).copy()).view(tdt)
    return out
