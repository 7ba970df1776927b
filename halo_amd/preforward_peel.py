"""``install_preforward_peel`` under the reference's module name
(halo/preforward_peel.py); the implementation is in ``chunked_prefill``."""
from .chunked_prefill import PreforwardPeelResult, install_preforward_peel  # noqa: F401

__all__ = ["install_preforward_peel", "PreforwardPeelResult"]
