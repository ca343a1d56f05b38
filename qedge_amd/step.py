"""Decode-step bookkeeping on the device: pending next-token slots, stop check, history.

The reference publishes each sampled id into a fixed GPU slot that the next
decode step reads as its input (``ModelRunner._publish_sample_ids``,
src/compute/model_runner.py:95-115), copies the ids to a pinned host buffer on a
side stream and waits for that copy (``_read_sample_ids``, :122-135), and then
``Scheduler.postprocess`` appends the token and checks EOS / length on the host
(src/control/scheduler.py:304-322).  ``DecodeStep`` does all of it in one
kernel after the sampler (``qs_step_finish``), so that sampler + bookkeeping can
be captured in the decode graph; the host reads the ids and finished flags from
host-mapped pinned buffers after one event.  With a token history, the sampled
ids are appended on the device (``qs_history_append``) instead of being
re-staged from the host every step.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _loaded_hip_runtime():
    """The HIP runtime this process already runs on (the one torch loaded), or None."""
    try:
        with open("/proc/self/maps") as f:
            paths = {line.split()[-1] for line in f if "libamdhip64" in line and "/" in line}
    except OSError:
        return None
    for path in sorted(paths):
        try:
            return ctypes.CDLL(path)  # already mapped: the same instance
        except OSError:
            continue
    return None


def _hip_device_pointer(host_tensor: torch.Tensor) -> int | None:
    """Device address of a pinned host tensor (hipHostGetDevicePointer), or None."""
    hip = _loaded_hip_runtime()
    if hip is None:
        return None
    dptr = ctypes.c_void_p()
    rc = hip.hipHostGetDevicePointer(ctypes.byref(dptr), ctypes.c_void_p(host_tensor.data_ptr()), ctypes.c_uint(0))
    return dptr.value if rc == 0 and dptr.value else None


class DecodeStep:
    """Device-resident per-row decode state for up to ``max_bs`` rows.

    ``pending``        int64 [n_pending]: the fixed next-token slots (model_runner.py:35-37)
    ``num_generated``  int32 [max_bs]: completion tokens per row
    ``min_tokens`` / ``max_tokens`` / ``ignore_eos``: the rows' stop parameters
    ``finished``       uint8 [max_bs]: set by ``finish``
    ``history`` / ``history_len``: optional token-history ring ([max_bs, H] int32) for the penalties
    ``host_ids`` / ``host_finished``: pinned host mirrors (``read``)
    """

    def __init__(self, max_bs: int, device: torch.device, *, n_pending: int | None = None, history: int = 0,
                 eos_id: int = -1) -> None:
        self.max_bs, self.device, self.eos_id = int(max_bs), torch.device(device), int(eos_id)
        n_pending = self.max_bs if n_pending is None else int(n_pending)
        if self.max_bs <= 0 or n_pending <= 0:
            raise ValueError("max_bs and n_pending must be positive")
        if history < 0 or history > _lib.QS_MAX_HISTORY:
            raise ValueError(f"history must be in [0, {_lib.QS_MAX_HISTORY}]")
        dev = self.device
        self.pending = torch.zeros(n_pending, dtype=torch.int64, device=dev)
        self.slots = torch.arange(self.max_bs, dtype=torch.int32, device=dev)
        self.num_generated = torch.zeros(self.max_bs, dtype=torch.int32, device=dev)
        self.min_tokens = torch.zeros(self.max_bs, dtype=torch.int32, device=dev)
        self.max_tokens = torch.ones(self.max_bs, dtype=torch.int32, device=dev)
        self.ignore_eos = torch.zeros(self.max_bs, dtype=torch.uint8, device=dev)
        self.finished = torch.zeros(self.max_bs, dtype=torch.uint8, device=dev)
        self.H = int(history)
        self.history = torch.full((self.max_bs, max(self.H, 1)), -1, dtype=torch.int32, device=dev)
        self.history_len = torch.zeros(self.max_bs, dtype=torch.int32, device=dev)
        self.host_ids = torch.zeros(self.max_bs, dtype=torch.int64, pin_memory=True)
        self.host_finished = torch.zeros(self.max_bs, dtype=torch.uint8, pin_memory=True)
        self._host_ids_dev = _hip_device_pointer(self.host_ids)
        self.copy_stream = torch.cuda.Stream(device=dev)
        self.event = torch.cuda.Event()

    # ---- host staging (once per admitted request, not per step)
    def set_row(self, r: int, *, slot: int | None = None, min_tokens: int = 0, max_tokens: int = 128,
                ignore_eos: bool = False, num_generated: int = 0, history: list[int] | None = None) -> None:
        """Stage row r's parameters (Sequence.from_prompt, src/data/sequence.py:99-128)."""
        if not 0 <= r < self.max_bs:
            raise IndexError(f"row {r} outside [0, {self.max_bs})")
        self.slots[r] = r if slot is None else int(slot)
        self.min_tokens[r] = int(min_tokens)
        self.max_tokens[r] = int(max_tokens)
        self.ignore_eos[r] = 1 if ignore_eos else 0
        self.num_generated[r] = int(num_generated)
        self.finished[r] = 0
        if self.H:
            ids = [] if history is None else [int(t) for t in history][-self.H:]
            row = torch.full((self.H,), -1, dtype=torch.int32)
            if ids:
                row[:len(ids)] = torch.tensor(ids, dtype=torch.int32)
            self.history[r].copy_(row)
            self.history_len[r] = len(ids)

    # ---- device work (capturable: allocates nothing, no host synchronisation)
    def finish(self, ids: torch.Tensor, B: int, *, append_history: bool = True) -> None:
        """Publish ``ids[:B]`` to their slots, count them, set ``finished``, append the history."""
        if ids.dtype != torch.int64 or ids.device != self.device or ids.numel() < B or not ids.is_contiguous():
            raise ValueError("ids must be a contiguous int64 tensor of >= B entries on the step's device")
        if not 0 <= B <= self.max_bs:
            raise ValueError(f"B must be in [0, {self.max_bs}]")
        lib = _lib.load()
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        p = lambda t: ctypes.c_void_p(t.data_ptr())
        host = ctypes.c_void_p(self._host_ids_dev) if self._host_ids_dev else None
        _lib.check(lib.qs_step_finish(p(ids), B, p(self.slots), p(self.pending), self.pending.numel(),
                                      p(self.num_generated), p(self.min_tokens), p(self.max_tokens),
                                      p(self.ignore_eos), self.eos_id, p(self.finished), host, stream))
        if self.H and append_history:
            _lib.check(lib.qs_history_append(p(self.history), B, self.H, p(self.history_len), p(ids), None,
                                             stream))

    def history_view(self, B: int) -> tuple[torch.Tensor, torch.Tensor] | tuple[None, None]:
        """(history, history_len) for qs_sample's hist_ids / hist_len."""
        return (self.history[:B], self.history_len[:B]) if self.H else (None, None)

    # ---- host read-back (one event, as _read_sample_ids)
    def read(self, ids: torch.Tensor, B: int) -> tuple[list[int], list[bool]]:
        """Ids and finished flags of the last ``finish`` on the host."""
        current = torch.cuda.current_stream(self.device)
        self.copy_stream.wait_stream(current)
        with torch.cuda.stream(self.copy_stream):
            if self._host_ids_dev is None:
                self.host_ids[:B].copy_(ids[:B], non_blocking=True)
            self.host_finished[:B].copy_(self.finished[:B], non_blocking=True)
        self.event.record(self.copy_stream)
        self.event.synchronize()
        return self.host_ids[:B].tolist(), [bool(x) for x in self.host_finished[:B].tolist()]


def step_finish_reference(ids: list[int], num_generated: list[int], min_tokens: list[int], max_tokens: list[int],
                          ignore_eos: list[bool], eos_id: int) -> tuple[list[int], list[bool]]:
    """Host statement of the stop rule of Scheduler.postprocess (src/control/scheduler.py:304-322)."""
    n_out, fin = [], []
    for t, n, mn, mx, ign in zip(ids, num_generated, min_tokens, max_tokens, ignore_eos):
        if mx <= 0:
            n_out.append(n)
            fin.append(True)
            continue
        n += 1
        hit_eos = (not ign) and n >= mn and eos_id >= 0 and t == eos_id
        n_out.append(n)
        fin.append(hit_eos or n >= mx)
    return n_out, fin
