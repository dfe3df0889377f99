"""Helpers shared by the GPU parity tests (host <-> device, tolerances)."""
import numpy as np
import torch


def dev(a: np.ndarray) -> torch.Tensor:
    """numpy -> device tensor (uint16 travels as int16 bits)."""
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor, dtype=None) -> np.ndarray:
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def empty(n, dtype) -> torch.Tensor:
    return torch.empty(n, dtype=dtype, device="cuda")


def zeros_synced(n, dtype) -> torch.Tensor:
    """A zeroed device buffer whose fill has completed: torch.zeros runs on
    torch's current stream, and a context on a side stream that writes the
    buffer next (a step buffer) is not ordered after that fill."""
    t = torch.zeros(n, dtype=dtype, device="cuda")
    torch.cuda.current_stream().synchronize()
    return t


def assert_close(got, want, rtol, atol, what=""):
    """|got-want| <= atol + rtol*|want| elementwise (mod.rs:137-153 form)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    excess = np.abs(got - want) - rtol * np.abs(want)
    i = int(np.argmax(excess))
    assert excess.flat[i] <= atol, (
        f"{what}: element {i}: got {got.flat[i]!r} want {want.flat[i]!r} "
        f"(excess {excess.flat[i]:.3e} > atol {atol:.3e})")


def rel_err(got, want) -> float:
    """max |got-want| / max |want| (normwise relative error)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-300))


def sample_rows(n: int) -> np.ndarray:
    """parity_gemv.rs:59-66: the first 64 rows, ~97 spread rows, the last."""
    rows = list(range(min(n, 64)))
    rows += list(range(64, n, max(n // 97, 1)))
    rows.append(n - 1)
    return np.array(sorted(set(rows)), np.int64)
