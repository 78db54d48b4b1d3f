"""Host side of the fail-stop guard: deadlines, fault injection and error words.

Every inter-workgroup wait in the kernels polls under a deadline on the 100 MHz
``s_memrealtime`` clock, checking it and the launch's abort flag every 64 polls. A wait
that passes its deadline records ``1 + site`` in the guard block's error word, raises
the abort flag (every other wait then gives up), mirrors the word into a pinned host
word, and the launch drains to its end. The runtime raises on the host before the next
launch and on every ``check()``.

The reference stops a failed launch with a store to the null page, which takes the
process down (``sgl_amd_mono/common/guard.py:91-97``). Here the launch ends normally
and the host raises instead: a deliberate GPU fault is not an acceptable stop on a
shared MI355X node, and a launch that never runs on after a failed wait keeps the
same guarantee (no output of a failed step is used, because the host refuses to go
on). Deadline and fault-injection semantics follow ``guard.py:60-88``.
"""

from __future__ import annotations

import os
from typing import Optional

from . import _lib

CLOCK_HZ = 100_000_000
# the reference compares time in 2^8-tick units as 32-bit scalars (guard.py:60-66);
# the same bound keeps a deadline portable between the two
TICK_SHIFT = 8
MAX_DEADLINE_TICKS = (1 << 31 << TICK_SHIFT) - 1
FAULT_ENV = "SGLANG_AMD_MONO_FAULT_INJECT"


def deadline_ticks(seconds: float) -> int:
    """Seconds -> clock ticks; refuses a deadline the 32-bit check cannot hold
    (``guard.py:69-76``)."""
    ticks = int(seconds * CLOCK_HZ)
    if ticks <= 0:
        raise ValueError(f"a wait deadline must be positive, got {seconds} s")
    if ticks > MAX_DEADLINE_TICKS:
        raise ValueError(
            f"a {seconds} s wait deadline does not fit the wait's 32-bit check; "
            f"use at most {MAX_DEADLINE_TICKS // CLOCK_HZ} s"
        )
    return ticks


def watchdog_deadline(watchdog_timeout: float) -> float:
    """Half the server's watchdog, at most 60 s (``guard.py:4-14``)."""
    return min(watchdog_timeout / 2.0, 60.0)


def fault_injection(rank: int) -> Optional[tuple[int, int]]:
    """``SGLANG_AMD_MONO_FAULT_INJECT=rank:site[:after]`` -> (site, after) for this rank,
    else None (``guard.py:79-88``). Once ``after`` launches ran, the wait at ``site``
    never completes, so it times out."""
    spec = os.environ.get(FAULT_ENV, "")
    if not spec:
        return None
    r, site, after = (spec.split(":") + ["0", "0"])[:3]
    return (int(site or 0), int(after or 0)) if int(r) == rank else None


def describe(words) -> Optional[str]:
    """A failure message from the guard block's words (a sequence of ints), or None."""
    dl, peer, fault = (int(words[i]) for i in (_lib.GUARD_ERR_DEADLINE, _lib.GUARD_ERR_PEER,
                                                _lib.GUARD_ERR_FAULT))
    if not (dl or peer or fault):
        return None
    site = _lib.SITES.get(dl - 1, f"site {dl - 1}") if dl else "-"
    return (f"monokernel wait timed out at {site} (deadline word {dl}, peer {peer}, "
            f"fault-injected {fault})")
