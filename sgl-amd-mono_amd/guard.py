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
on). The fault-injection variable and its format are the reference's (``guard.py:79-88``).
"""

from __future__ import annotations

import os
from typing import Optional

from . import _lib

CLOCK_HZ = 100_000_000  # s_memrealtime ticks a second
# the kernels compare 64-bit tick differences, so any deadline fits; an hour bounds it
# far above every server watchdog, so a larger value is a configuration mistake
MAX_DEADLINE_S = 3600.0
FAULT_ENV = "SGLANG_AMD_MONO_FAULT_INJECT"


def deadline_ticks(seconds: float) -> int:
    """A wait deadline in clock ticks; ``ValueError`` outside (0, MAX_DEADLINE_S]."""
    if not 0.0 < float(seconds) <= MAX_DEADLINE_S:
        raise ValueError(f"wait deadline {seconds!r} s: must lie in (0, {MAX_DEADLINE_S:g}] s")
    return max(1, int(float(seconds) * CLOCK_HZ))


def watchdog_deadline(watchdog_timeout: float) -> float:
    """Half the server's watchdog, at most 60 s (``guard.py:4-14``)."""
    return min(watchdog_timeout / 2.0, 60.0)


def fault_injection(rank: int) -> Optional[tuple[int, int]]:
    """The test fault injection ``SGLANG_AMD_MONO_FAULT_INJECT=rank:site[:after]`` (the
    reference's variable and format, ``guard.py:79-88``) for ``rank``: (site, after), or
    None when unset or meant for another rank. Once ``after`` launches ran on a runtime,
    its wait at ``site`` never completes and times out."""
    raw = os.environ.get(FAULT_ENV, "").strip()
    if not raw:
        return None
    fields = raw.split(":")
    if len(fields) not in (2, 3) or not all(f.strip().lstrip("-").isdigit() for f in fields):
        raise ValueError(f"{FAULT_ENV}={raw!r}: expected rank:site or rank:site:after")
    who, site = int(fields[0]), int(fields[1])
    after = int(fields[2]) if len(fields) == 3 else 0
    return (site, after) if who == rank else None


def describe(words) -> Optional[str]:
    """A failure message from the guard block's words (a sequence of ints), or None."""
    dl, peer, fault = (int(words[i]) for i in (_lib.GUARD_ERR_DEADLINE, _lib.GUARD_ERR_PEER,
                                                _lib.GUARD_ERR_FAULT))
    if not (dl or peer or fault):
        return None
    site = _lib.SITES.get(dl - 1, f"site {dl - 1}") if dl else "-"
    return (f"monokernel wait timed out at {site} (deadline word {dl}, peer {peer}, "
            f"fault-injected {fault})")
