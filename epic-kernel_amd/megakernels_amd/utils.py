"""Small helpers shared by the scheduler and the launcher.

Counterparts of ``megakernels/utils.py:125-135`` (``get_sm_count``) and the
``assert_div`` helper the Mixtral scheduler imports (``megakernels/mixtral/
scheduler.py:19``).
"""

from __future__ import annotations

import torch


def assert_div(a: int, b: int) -> int:
    """Return ``a // b`` and fail loudly when ``b`` does not divide ``a``."""
    if b <= 0 or a % b != 0:
        raise ValueError(f"{a} is not divisible by {b}")
    return a // b


def get_sm_count(device) -> int:
    """Number of compute units on ``device`` (256 on an MI355X).

    Same contract as the reference (``megakernels/utils.py:133-135``): the
    count of independent workers the persistent kernel is launched with.
    """
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(
            f"get_sm_count needs a GPU device, got {dev}; set "
            "globs.sm_count_override for CPU-only scheduling"
        )
    return torch.cuda.get_device_properties(dev).multi_processor_count
