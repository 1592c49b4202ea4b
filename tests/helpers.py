"""Small helpers shared by the test modules.

The parity bar for 16-bit outputs is "within ``atol`` before one correct
rounding to the output dtype": an output passes when it is the round-to-
nearest of some value within ``atol`` of the float64 reference, that is when

    |got - ref| <= atol + 1/2 ulp(|ref| + atol)

(the half ulp is taken at the largest magnitude the pre-rounding value can
have, so a reference just below a power of two is not held to the finer
spacing of its own binade).  For bf16 at |o| in [1, 2) that allows 2e-3 +
3.9e-3 = 5.9e-3; below |o| = 2^-4 it is within 1.2e-4 of atol itself.
"""

from __future__ import annotations


def announce(msg: str) -> None:
    """Print and flush which case a GPU step is about to run."""
    print(f"[case] {msg}", flush=True)


def f64(t):
    """A tensor as a float64 numpy array on the host."""
    import numpy as np

    return t.detach().float().cpu().numpy().astype(np.float64)


_MANT = {"bfloat16": 7, "float16": 10, "float32": 23}


def _mant(dtype) -> int:
    return _MANT[str(dtype).replace("torch.", "")]


def ulp(x, dtype):
    """One unit in the last place of ``dtype`` at the magnitude of each element of x."""
    import numpy as np

    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -24)))
    return 2.0 ** (e - _mant(dtype))


def allowed_error(ref, dtype, atol: float):
    """The elementwise bar: ``atol`` before one round-to-nearest into ``dtype``."""
    import numpy as np

    return atol + 0.5 * ulp(np.abs(ref) + atol, dtype)


def assert_close(got, ref, atol: float, what: str, dtype=None) -> float:
    """Every element of ``got`` within ``atol`` of ``ref`` before one output rounding.

    ``got`` is a tensor (its dtype is the output dtype) or a float64 array
    with ``dtype`` given.  Returns the max abs error.
    """
    import numpy as np

    if dtype is None:
        dtype = got.dtype
    g = got if isinstance(got, np.ndarray) else f64(got)
    assert g.shape == ref.shape, (g.shape, ref.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - ref)
    allowed = allowed_error(ref, dtype, atol)
    worst = np.unravel_index(np.argmax(err - allowed), err.shape)
    assert (err <= allowed).all(), (
        f"{what}: max err {err.max():.3e} (at {worst}: got {g[worst]:.6f} ref {ref[worst]:.6f}, "
        f"allowed {allowed[worst]:.2e})")
    return float(err.max())
