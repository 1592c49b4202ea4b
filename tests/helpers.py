"""Small helpers shared by the test modules."""

from __future__ import annotations


def announce(msg: str) -> None:
    """Print and flush which case a GPU step is about to run."""
    print(f"[case] {msg}", flush=True)
