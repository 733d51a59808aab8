"""The Spar tensor/ops API of the HIP backend, from Python.

Re-exports the pybind11 binding of the C++ host library (spar_amd/_spar*.so).
Importing fails loudly when the extension has not been built.
"""
try:
    from spar_amd._spar import *  # noqa: F401,F403
    from spar_amd._spar import LogicError  # noqa: F401
except ImportError as error:  # pragma: no cover - exercised only when unbuilt
    raise ImportError("spar_amd._spar is not built; run `python -m spar_amd.build`") from error
