"""MI355X (gfx950) FP8 mixture-of-experts decode layer.

Python host code on PyTorch-ROCm drives hand-written HIP kernels through the C
ABI declared in include/megamoe.h (libmegamoe.so, built in-tree by
``build.build_library``). ``submission.build(case)`` is the reference
harness's ``build(case) -> run(inputs)`` drop-in.
"""

from . import cases, workloads  # noqa: F401
from .cases import CASES, Case, case, development  # noqa: F401
