"""Small helpers shared by the test modules."""

from __future__ import annotations


def announce(msg: str) -> None:
    """Print and flush which case a GPU step is about to run."""
    print(f"[case] {msg}", flush=True)


def f64(t):
    """A tensor as a float64 numpy array on the host."""
    import numpy as np

    return t.detach().float().cpu().numpy().astype(np.float64)


def ulp(x, dtype):
    """One unit in the last place of ``dtype`` at the magnitude of each element of x."""
    import numpy as np
    import torch

    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[dtype]
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -24)))
    return 2.0 ** (e - mant)


def assert_close(got, ref, atol: float, what: str) -> float:
    """max |got - ref| <= max(atol, one output ulp of |ref|) elementwise; returns the max error."""
    import numpy as np

    g = f64(got)
    assert g.shape == ref.shape, (g.shape, ref.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - ref)
    allowed = np.maximum(atol, ulp(ref, got.dtype))
    worst = np.unravel_index(np.argmax(err - allowed), err.shape)
    assert (err <= allowed).all(), (
        f"{what}: max err {err.max():.3e} (at {worst}: got {g[worst]:.6f} ref {ref[worst]:.6f}, "
        f"allowed {allowed[worst]:.2e})")
    return float(err.max())
