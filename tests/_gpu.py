"""Helpers for the GPU tests: device buffers (torch is used only for device memory and
synchronisation), descriptors over them, and the parity bar."""
import numpy as np
import torch

import cvattn

MAX_ABS = 2e-3   # attention parity bar vs the fp64 oracle (at least fp32-accumulation accurate)
MEAN_ABS = 2e-4


def dev(a: np.ndarray) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to("cuda:0")


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def empty_f32(*shape) -> torch.Tensor:
    return torch.full(shape, float("nan"), dtype=torch.float32, device="cuda:0")


def workspace(nbytes: int) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device="cuda:0")


def check_close(got: np.ndarray, want: np.ndarray, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    mx, mn = float(err.max()) if err.size else 0.0, float(err.mean()) if err.size else 0.0
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3g} mean-abs {mn:.3g}"
    return mx, mn


def run_fa(eng, q, k, v, mask, dst, scale=0.125):
    ws_bytes = eng.flash_attn_ext_workspace(q, k, v, mask)
    ws = workspace(ws_bytes)
    rc = eng.flash_attn_ext(q, k, v, mask, dst, scale, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK, eng.status_string(rc)
    torch.cuda.synchronize()
    return ws
