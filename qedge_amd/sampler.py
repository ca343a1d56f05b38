"""BatchSampler on the MI355X HIP kernels.

Drop-in for the reference's ``BatchSampler`` (src/compute/sampler.py:22-41):
same ``forward(logits, temperatures, top_ps, *, all_greedy, use_top_p)``
signature and int64 ``[B]`` result, plus keyword-only extensions (top-k, min_p,
penalties over a token history, host uniforms, a dispatch order).  Every call
goes to ``libqsampler.so``; there is no PyTorch fallback.
"""
from __future__ import annotations

import ctypes

import torch
from torch import nn

from . import _lib

_DTYPES = {torch.float32: _lib.QS_DTYPE_F32, torch.bfloat16: _lib.QS_DTYPE_BF16}
# From this many rows (and no top-k), one workgroup per row beats cooperating
# workgroups: the batch alone fills the GPU.
SOLO_MIN_ROWS = 512


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class Workspace:
    """Device workspace for batches of up to ``max_bs`` rows of ``V`` logits.

    Zeroed once; every call leaves it zeroed again.  One workspace serves any
    batch size up to ``max_bs`` (the fixed buffers of src/data/batch.py:57-66).
    """

    def __init__(self, max_bs: int, V: int, dtype: torch.dtype, H: int, device: torch.device):
        lib = _lib.load()
        self.max_bs, self.V, self.device = int(max_bs), int(V), torch.device(device)
        self.nbytes = int(lib.qs_workspace_bytes(self.max_bs, self.V, _DTYPES[dtype], int(H)))
        if self.nbytes == 0:
            raise ValueError(f"no workspace layout for max_bs={max_bs}, V={V}")
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=self.device)
        _lib.check(lib.qs_workspace_init(ctypes.c_void_p(self.buf.data_ptr()), self.nbytes,
                                         ctypes.c_void_p(_stream_handle(self.device))))

    def fits(self, B: int, V: int, H: int = 0) -> bool:
        return B <= self.max_bs and V == self.V


def _vec(t: torch.Tensor | None, B: int, dtype: torch.dtype, name: str, device: torch.device) -> int | None:
    """Pointer of a contiguous ``dtype`` vector of at least B entries on ``device``."""
    if t is None:
        return None
    if t.dtype != dtype or t.dim() != 1 or t.shape[0] < B or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} tensor of >= {B} entries")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, the logits on {device}")
    return t.data_ptr()


def sample_into(logits: torch.Tensor, out_ids: torch.Tensor, workspace: Workspace, *,
                temperatures: torch.Tensor | None, top_ps: torch.Tensor | None = None,
                top_ks: torch.Tensor | None = None, min_ps: torch.Tensor | None = None,
                repetition_penalties: torch.Tensor | None = None,
                presence_penalties: torch.Tensor | None = None,
                frequency_penalties: torch.Tensor | None = None, history: torch.Tensor | None = None,
                history_len: torch.Tensor | None = None, uniforms: torch.Tensor | None = None,
                row_order: torch.Tensor | None = None, all_greedy: bool = False, use_top_p: bool = False,
                out_probs: torch.Tensor | None = None, out_kept: torch.Tensor | None = None,
                no_wait: bool = False, solo: bool | None = None) -> torch.Tensor:
    """Sample into caller-owned ``out_ids`` (int64 [B]); allocates nothing.

    Every tensor must be on the logits' device; sizes and dtypes are checked
    here (ValueError) so that no kernel reads or writes outside a buffer.
    ``solo`` resolves every row by one workgroup (QS_FLAG_SOLO); by default it
    is used for batches of at least SOLO_MIN_ROWS rows without top-k.
    """
    if logits.dim() != 2 or logits.dtype not in _DTYPES or not logits.is_cuda:
        raise ValueError("logits must be a [B, V] float32/bfloat16 device tensor")
    if logits.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    dev = logits.device
    B, V = logits.shape
    if not workspace.fits(B, V):
        raise ValueError(f"workspace serves up to {workspace.max_bs} rows of V={workspace.V}, got [{B}, {V}]")
    if workspace.device != dev:
        raise ValueError("workspace is on another device")
    if out_ids.dtype != torch.int64 or out_ids.dim() != 1 or out_ids.numel() < B or not out_ids.is_contiguous():
        raise ValueError("out_ids must be a contiguous int64 tensor of >= B entries")
    if out_ids.device != dev:
        raise ValueError("out_ids must be on the logits' device")
    if not all_greedy and temperatures is None:
        raise ValueError("temperatures are required unless all_greedy")
    H = 0
    if history is not None:
        if history.dtype != torch.int32 or history.dim() != 2 or history.shape[0] < B or not history.is_contiguous():
            raise ValueError("history must be a contiguous int32 [>= B, H] tensor")
        if history.device != dev:
            raise ValueError("history must be on the logits' device")
        H = int(history.shape[1])
        if H > _lib.QS_MAX_HISTORY:
            raise ValueError(f"history longer than {_lib.QS_MAX_HISTORY} ids")
        if H == 0:
            history = None
    if history_len is not None and history is None:
        raise ValueError("history_len needs history")
    if out_probs is not None:
        if (out_probs.dtype != torch.float32 or out_probs.dim() != 2 or out_probs.shape[0] < B
                or out_probs.shape[1] != V or not out_probs.is_contiguous() or out_probs.device != dev):
            raise ValueError("out_probs must be a contiguous float32 [>= B, V] tensor on the logits' device")
    if solo is None:
        solo = B >= SOLO_MIN_ROWS and top_ks is None
    flags = ((_lib.QS_FLAG_ALL_GREEDY if all_greedy else 0) | (_lib.QS_FLAG_USE_TOP_P if use_top_p else 0)
             | (_lib.QS_FLAG_NO_WAIT if no_wait else 0) | (_lib.QS_FLAG_SOLO if solo else 0))
    f32, i32 = torch.float32, torch.int32
    args = (
        ctypes.c_void_p(logits.data_ptr()), logits.stride(0), _DTYPES[logits.dtype], B, V,
        _vec(temperatures, B, f32, "temperatures", dev), _vec(top_ps, B, f32, "top_ps", dev),
        _vec(top_ks, B, i32, "top_ks", dev), _vec(min_ps, B, f32, "min_ps", dev),
        _vec(repetition_penalties, B, f32, "repetition_penalties", dev),
        _vec(presence_penalties, B, f32, "presence_penalties", dev),
        _vec(frequency_penalties, B, f32, "frequency_penalties", dev),
        None if history is None else history.data_ptr(), H, _vec(history_len, B, i32, "history_len", dev),
        _vec(uniforms, B, f32, "uniforms", dev), _vec(row_order, B, i32, "row_order", dev), flags,
        ctypes.c_void_p(out_ids.data_ptr()), None if out_probs is None else out_probs.data_ptr(),
        _vec(out_kept, B, i32, "out_kept", dev), ctypes.c_void_p(workspace.buf.data_ptr()), workspace.nbytes,
        ctypes.c_void_p(_stream_handle(dev)))
    _lib.check(_lib.load().qs_sample(*args))
    return out_ids


class BatchSampler(nn.Module):
    """Batched greedy / temperature / top-k / min_p / top-p sampling with history penalties.

    Mirrors src/compute/sampler.py:25-41.  ``all_greedy`` and ``use_top_p`` are
    the host flags the reference derives from the CPU-side parameters
    (src/compute/model_runner.py:82-83); ``use_top_p=False`` ignores top_ps as
    the reference does.  ``uniforms`` (float32 [B] in [0, 1)) are the host's
    seeded draws; when omitted they come from torch's generator on the device.

    One workspace per (device, V), sized for ``max_bs`` rows (grown to the
    largest batch seen when ``max_bs`` is not given), serves every batch size.
    """

    def __init__(self, max_bs: int | None = None) -> None:
        super().__init__()
        self.max_bs = max_bs
        self._ws: dict[tuple, Workspace] = {}

    def workspace(self, B: int, V: int, dtype: torch.dtype, device: torch.device) -> Workspace:
        key = (torch.device(device), V)
        ws = self._ws.get(key)
        if ws is None or not ws.fits(B, V):
            if self.max_bs is not None and B > self.max_bs:
                raise ValueError(f"batch of {B} rows exceeds max_bs={self.max_bs}")
            size = self.max_bs if self.max_bs is not None else max(B, 2 * ws.max_bs if ws is not None else B)
            ws = Workspace(size, V, dtype, 0, device)
            self._ws[key] = ws
        return ws

    def forward(self, logits: torch.Tensor, temperatures: torch.Tensor, top_ps: torch.Tensor, *,
                all_greedy: bool = False, use_top_p: bool = False, top_ks: torch.Tensor | None = None,
                min_ps: torch.Tensor | None = None, repetition_penalties: torch.Tensor | None = None,
                presence_penalties: torch.Tensor | None = None,
                frequency_penalties: torch.Tensor | None = None, history: torch.Tensor | None = None,
                history_len: torch.Tensor | None = None, uniforms: torch.Tensor | None = None,
                row_order: torch.Tensor | None = None) -> torch.Tensor:
        B, V = logits.shape
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        if uniforms is None and not all_greedy:
            uniforms = torch.rand(B, device=logits.device, dtype=torch.float32)
        ws = self.workspace(B, V, logits.dtype, logits.device)
        out = torch.empty(B, dtype=torch.int64, device=logits.device)
        sl = lambda t: None if t is None else t[:B]
        return sample_into(logits, out, ws, temperatures=sl(temperatures), top_ps=sl(top_ps), top_ks=sl(top_ks),
                           min_ps=sl(min_ps), repetition_penalties=sl(repetition_penalties),
                           presence_penalties=sl(presence_penalties), frequency_penalties=sl(frequency_penalties),
                           history=None if history is None else history[:B], history_len=sl(history_len),
                           uniforms=sl(uniforms), row_order=sl(row_order), all_greedy=all_greedy,
                           use_top_p=use_top_p)


def argmax_into(logits: torch.Tensor, out_ids: torch.Tensor, workspace: Workspace) -> torch.Tensor:
    """First index of the row maximum (NaN is maximum) into ``out_ids``.

    Replaces ``logits.argmax(-1)`` on the all-greedy path and in the captured
    decode graph (src/compute/model_runner.py:85,353).
    """
    if logits.dim() != 2 or logits.dtype not in _DTYPES or not logits.is_cuda or logits.stride(1) != 1:
        raise ValueError("logits must be a [B, V] float32/bfloat16 device tensor with contiguous rows")
    B, V = logits.shape
    if not workspace.fits(B, V):
        raise ValueError("workspace too small for this batch")
    if out_ids.dtype != torch.int64 or out_ids.numel() < B or out_ids.device != logits.device:
        raise ValueError("out_ids must be int64 [>= B] on the logits' device")
    lib = _lib.load()
    _lib.check(lib.qs_argmax(ctypes.c_void_p(logits.data_ptr()), logits.stride(0), _DTYPES[logits.dtype], B, V,
                             ctypes.c_void_p(out_ids.data_ptr()), ctypes.c_void_p(workspace.buf.data_ptr()),
                             workspace.nbytes, ctypes.c_void_p(_stream_handle(logits.device))))
    return out_ids


def sample_gpu(sampler: "BatchSampler", logits: torch.Tensor | list[torch.Tensor], batch) -> torch.Tensor:
    """One token per row: the role of ModelRunner._sample_gpu (src/compute/model_runner.py:77-93).

    ``logits`` is a [B, V] tensor or a list of [1, V] rows (concatenated as at
    model_runner.py:81); ``batch`` is a filled ``SamplingBatch`` whose host flags
    pick the path: all-greedy rows without penalties take the argmax kernel
    (model_runner.py:84-85); everything else, greedy rows with penalties
    included, runs the sampler with the batch's device buffers (:87-92).
    """
    if isinstance(logits, (list, tuple)):
        if not logits:
            return torch.empty(0, dtype=torch.long, device=batch.device)
        logits = torch.cat(list(logits), dim=0)
    B, V = logits.shape
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    if batch.all_greedy and not batch.use_penalties:
        ws = sampler.workspace(B, V, logits.dtype, logits.device)
        out = torch.empty(B, dtype=torch.int64, device=logits.device)
        return argmax_into(logits, out, ws)
    kw = batch.sampler_kwargs()
    return sampler(logits, kw.pop("temperatures"), kw.pop("top_ps"), **kw)


_default = None


def _default_sampler() -> BatchSampler:
    global _default
    if _default is None:
        _default = BatchSampler()
    return _default


@torch.library.custom_op("qedge_amd::sample", mutates_args=())
def sample_op(logits: torch.Tensor, temperatures: torch.Tensor, top_ps: torch.Tensor, top_ks: torch.Tensor,
              min_ps: torch.Tensor, repetition_penalties: torch.Tensor, presence_penalties: torch.Tensor,
              frequency_penalties: torch.Tensor, history: torch.Tensor, history_len: torch.Tensor,
              uniforms: torch.Tensor, all_greedy: bool, use_top_p: bool) -> torch.Tensor:
    """Custom-op boundary for compiled callers (pattern of src/compute/layers/ops.py:18-39).

    Every extension is a tensor argument: a history of shape [B, 0] means no
    penalties (and history_len is then ignored)."""
    hist = history if history.numel() > 0 else None
    return _default_sampler()(logits, temperatures, top_ps, all_greedy=all_greedy, use_top_p=use_top_p,
                              top_ks=top_ks, min_ps=min_ps, repetition_penalties=repetition_penalties,
                              presence_penalties=presence_penalties, frequency_penalties=frequency_penalties,
                              history=hist, history_len=history_len if hist is not None else None,
                              uniforms=uniforms)


@sample_op.register_fake
def _sample_op_fake(logits, temperatures, top_ps, top_ks, min_ps, repetition_penalties, presence_penalties,
                    frequency_penalties, history, history_len, uniforms, all_greedy, use_top_p):
    return torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
