"""Helpers for the GPU parity tests (inputs from the oracle's seeded generator)."""
import numpy as np
import torch

import oracle as O

D = 128
# Attention outputs vs the fp32 oracle (fp16 outputs): the north-star tolerance.
MAX_ABS_TOL = 1e-2
MEAN_ABS_TOL = 1e-3


def dev(a_u16: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a_u16).view(np.float16)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy().view(np.uint16)


def host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def normal(tag: str, shape):
    return O.fill_normal_f16(O.seed_for(tag), shape)


def gamma(tag: str):
    return O.fill_uniform_f16(O.seed_for(tag), 0.8, 1.2, D)


def assert_close(got: np.ndarray, ref: np.ndarray, what: str):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    mx, mean = float(err.max()), float(err.mean())
    print(f"[{what}] max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert mx <= MAX_ABS_TOL, f"{what}: max_abs {mx:.3e} > {MAX_ABS_TOL}"
    assert mean <= MEAN_ABS_TOL, f"{what}: mean_abs {mean:.3e} > {MEAN_ABS_TOL}"
