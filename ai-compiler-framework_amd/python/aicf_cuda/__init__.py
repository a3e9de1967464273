"""aicf_cuda: the gfx950 backend behind the reference's `aicf_cuda._C` API.

`import torch` must come first: torch ships its own HIP runtime, and loading
it before libaicf_hip.so makes both share that one runtime.  The native
module is required; there is no fallback path.
"""
import torch  # noqa: F401  (loads torch's HIP runtime first)

from . import _C  # noqa: E402

__all__ = ["_C"]
