"""A monokernel runtime: the scratch, guard block and host error word one launch kind
owns, on one device.

Mirrors the ownership of ``Glm53Runtime`` (``sgl_amd_mono/glm53/gfx950/runner.py:133-215``):
the runtime allocates the hand-off scratch and the epoch/guard block once; the caller
owns every weight, cache and step table. Launches reuse the same scratch, so launches
of one runtime must be stream-ordered (they are: one stream per rank).

Nothing here has to run between launches: each launch's last CTA clears one 16 KiB
chunk of the scratch in turn (so no tagged pair outlives the tag cycle; the reference
runs a scrub kernel after each step for this, deepseek_v4/gfx950/kernels/layer.py:843-895),
and a launch that failed, or follows a failure on the same guard block, fills its outputs
with NaN before it ends, so a replayed graph cannot turn a failed step into tokens. The
host reads the error word when it can (``check``, ``before_launch``) and ``reset``s.
"""

from __future__ import annotations

import torch

from . import _lib, guard


def shared_or_new(rt, scratch_bytes: int, device, deadline_s: float) -> "MonoRuntime":
    """``rt`` when it is given (a runtime shared by the stream-ordered launches of many
    layers; its scratch must be at least ``scratch_bytes``), else a runtime of its own."""
    if rt is None:
        return MonoRuntime(scratch_bytes, device, deadline_s)
    if rt.device != torch.device(device) or rt.scratch.numel() < scratch_bytes:
        raise ValueError(f"a shared runtime on {rt.device} with {rt.scratch.numel()} B of "
                         f"scratch cannot serve a launch needing {scratch_bytes} B on {device}")
    return rt


class MonoRuntime:
    """Scratch + guard of one launch kind on ``device``."""

    def __init__(self, scratch_bytes: int, device, deadline_s: float = 10.0):
        import torch

        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("a monokernel runtime lives on a GPU")
        info = _lib.MonoDeviceInfo()
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().mono_device_info(self.device.index or 0, info), "device info")
            if not info.is_gfx950:
                raise RuntimeError("the monokernels need a gfx950 (MI355X) device")
            self.grid = info.grid
            scratch_bytes = (int(scratch_bytes) + 255) & ~255
            self.scratch = torch.zeros(scratch_bytes, dtype=torch.uint8, device=self.device)
            self.guard = torch.zeros(_lib.GUARD_WORDS, dtype=torch.int32, device=self.device)
            # pinned host mirror of the first failure (written by the kernel, read here
            # without a device synchronisation)
            self.host_error = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.set_deadline(deadline_s)

    # ------------------------------------------------------------------ guard
    def set_deadline(self, seconds: float) -> None:
        guard.deadline_ticks(seconds)  # validates
        with torch.cuda.device(self.device):
            _lib.check(
                _lib.lib().mono_set_deadline(self.guard.data_ptr(), float(seconds),
                                             _lib.stream_handle()),
                "set deadline",
            )
        self.deadline_s = seconds

    def failed(self):
        """A failure message if a launch of this runtime timed out, else None (no sync)."""
        site = int(self.host_error[0])
        if site:
            return guard.describe([0, 0, 0, site, 0, 0] + [0] * 10) or f"failed (site {site})"
        return None

    def check(self, sync: bool = True) -> None:
        """Raise if a launch failed; with ``sync`` read the device guard words too."""
        if sync:
            torch.cuda.synchronize(self.device)
            msg = guard.describe(self.guard.cpu().tolist())
            if msg:
                raise RuntimeError(msg)
        msg = self.failed()
        if msg:
            raise RuntimeError(msg)

    def before_launch(self) -> None:
        """Refuse to launch after a failure (a launch would only write NaN)."""
        msg = self.failed()
        if msg:
            raise RuntimeError(f"{msg}; reset() the runtime before launching again")

    def reset(self, keep_error: bool = False) -> None:
        """Zero the scratch and the guard words (the deadline stays)."""
        with torch.cuda.device(self.device):
            _lib.check(
                _lib.lib().mono_reset(self.scratch.data_ptr(), self.scratch.numel(),
                                      self.guard.data_ptr(), _lib.stream_handle()),
                "reset",
            )
        if not keep_error:
            self.host_error.zero_()
