"""Input builders shared by the CPU and GPU tests."""

from __future__ import annotations

import numpy as np
import torch

from oracle.update import pack


def reference_init(out_features: int, in_features: int, max_code: int,
                   weight: torch.Tensor | None = None):
    """Codes and scales as DiscreteRatchetLinear.__init__ derives them from a float matrix
    (ratchet.py:369-386): kaiming-uniform draw from the global torch RNG when no weight
    is given, per-row absmax scale, round, clamp. Returns (code int8, scale float32)."""
    if weight is None:
        ref = torch.empty(out_features, in_features, dtype=torch.float32)
        torch.nn.init.kaiming_uniform_(ref, a=5**0.5)
    else:
        ref = weight.detach().float().cpu()
    row_max = ref.abs().amax(dim=1)
    scale = (row_max / max_code).clamp_min(torch.finfo(torch.float32).eps)
    code = torch.round(ref / scale[:, None]).clamp(-max_code, max_code)
    return code.to(torch.int8).numpy(), scale.numpy()


def synthetic_state(rows: int, cols: int, max_code: int, seed: int,
                    random_pressure: bool = True):
    """Uniform codes in [-max_code, max_code], pressure uniform in [-7, 7] (or 0),
    row scales U[0.02, 0.1]. Returns (packed uint8, scale float32)."""
    rng = np.random.default_rng(seed)
    code = rng.integers(-max_code, max_code + 1, size=(rows, cols), dtype=np.int8)
    if random_pressure:
        pressure = rng.integers(-7, 8, size=(rows, cols), dtype=np.int8)
    else:
        pressure = np.zeros((rows, cols), np.int8)
    scale = rng.uniform(0.02, 0.1, size=rows).astype(np.float32)
    return pack(code, pressure, max_code), scale
