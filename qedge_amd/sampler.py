"""BatchSampler on the MI355X HIP kernels.

Drop-in for the reference's ``BatchSampler`` (src/compute/sampler.py:22-41):
same ``forward(logits, temperatures, top_ps, *, all_greedy, use_top_p)``
signature and int64 ``[B]`` result, plus keyword-only extensions (top-k,
penalties over a token history, host uniforms).  Every call goes to
``libqsampler.so``; there is no PyTorch fallback.
"""
from __future__ import annotations

import ctypes

import torch
from torch import nn

from . import _lib

_DTYPES = {torch.float32: _lib.QS_DTYPE_F32, torch.bfloat16: _lib.QS_DTYPE_BF16}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class Workspace:
    """Device workspace for one (B, V, H) shape; zeroed once, self-cleaning after."""

    def __init__(self, B: int, V: int, dtype: torch.dtype, H: int, device: torch.device):
        lib = _lib.load()
        self.key = (B, V, H)
        self.nbytes = int(lib.qs_workspace_bytes(B, V, _DTYPES[dtype], H))
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=device)
        _lib.check(lib.qs_workspace_init(ctypes.c_void_p(self.buf.data_ptr()), self.nbytes,
                                         ctypes.c_void_p(_stream_handle(device))))

    def fits(self, B: int, V: int, H: int) -> bool:
        return self.key == (B, V, H)


def _f32(t: torch.Tensor | None, B: int, name: str) -> torch.Tensor | None:
    if t is None:
        return None
    if t.dtype != torch.float32 or t.dim() != 1 or t.shape[0] < B or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 [>= B] tensor")
    return t


def sample_into(logits: torch.Tensor, out_ids: torch.Tensor, workspace: Workspace, *,
                temperatures: torch.Tensor | None, top_ps: torch.Tensor | None = None,
                top_ks: torch.Tensor | None = None, repetition_penalties: torch.Tensor | None = None,
                presence_penalties: torch.Tensor | None = None,
                frequency_penalties: torch.Tensor | None = None, history: torch.Tensor | None = None,
                uniforms: torch.Tensor | None = None, all_greedy: bool = False, use_top_p: bool = False,
                mass_rows: bool = True, out_probs: torch.Tensor | None = None,
                out_kept: torch.Tensor | None = None) -> torch.Tensor:
    """Sample into caller-owned ``out_ids`` (int64 [B]); allocates nothing.

    ``mass_rows`` is a host-side batch flag from the CPU parameters: False when
    every sampling row has 0 < top_k <= QS_TOPK_FAST_MAX, which skips the launch
    that serves top-k-off rows (such a row is still resolved exactly if present).
    """
    if logits.dim() != 2 or logits.dtype not in _DTYPES or not logits.is_cuda:
        raise ValueError("logits must be a [B, V] float32/bfloat16 device tensor")
    if logits.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    B, V = logits.shape
    H = 0 if history is None else int(history.shape[1])
    if not workspace.fits(B, V, H):
        raise ValueError("workspace shape mismatch")
    if out_ids.dtype != torch.int64 or out_ids.numel() < B:
        raise ValueError("out_ids must be int64 [>= B]")
    if top_ks is not None and (top_ks.dtype != torch.int32 or not top_ks.is_contiguous()):
        raise ValueError("top_ks must be contiguous int32")
    if history is not None and (history.dtype != torch.int32 or not history.is_contiguous()):
        raise ValueError("history must be contiguous int32 [B, H]")
    flags = ((_lib.QS_FLAG_ALL_GREEDY if all_greedy else 0) | (_lib.QS_FLAG_USE_TOP_P if use_top_p else 0)
             | (0 if mass_rows else _lib.QS_FLAG_NO_MASS_ROWS))
    lib = _lib.load()
    rc = lib.qs_sample(
        ctypes.c_void_p(logits.data_ptr()), logits.stride(0), _DTYPES[logits.dtype], B, V,
        _ptr(_f32(temperatures, B, "temperatures")), _ptr(_f32(top_ps, B, "top_ps")), _ptr(top_ks),
        _ptr(_f32(repetition_penalties, B, "repetition_penalties")),
        _ptr(_f32(presence_penalties, B, "presence_penalties")),
        _ptr(_f32(frequency_penalties, B, "frequency_penalties")), _ptr(history), H,
        _ptr(_f32(uniforms, B, "uniforms")), flags, ctypes.c_void_p(out_ids.data_ptr()), _ptr(out_probs),
        _ptr(out_kept), ctypes.c_void_p(workspace.buf.data_ptr()), workspace.nbytes,
        ctypes.c_void_p(_stream_handle(logits.device)))
    _lib.check(rc)
    return out_ids


class BatchSampler(nn.Module):
    """Batched greedy / temperature / top-k / top-p sampling with history penalties.

    Mirrors src/compute/sampler.py:25-41.  ``all_greedy`` and ``use_top_p`` are
    the host flags the reference derives from the CPU-side parameters
    (src/compute/model_runner.py:82-83); ``use_top_p=False`` ignores top_ps as
    the reference does.  ``uniforms`` (float32 [B] in [0, 1)) are the host's
    seeded draws; when omitted they come from torch's generator on the device.
    """

    def __init__(self) -> None:
        super().__init__()
        self._ws: dict[tuple, Workspace] = {}

    def workspace(self, B: int, V: int, dtype: torch.dtype, H: int, device: torch.device) -> Workspace:
        key = (device, B, V, H)
        ws = self._ws.get(key)
        if ws is None:
            ws = Workspace(B, V, dtype, H, device)
            self._ws[key] = ws
        return ws

    def forward(self, logits: torch.Tensor, temperatures: torch.Tensor, top_ps: torch.Tensor, *,
                all_greedy: bool = False, use_top_p: bool = False, top_ks: torch.Tensor | None = None,
                repetition_penalties: torch.Tensor | None = None,
                presence_penalties: torch.Tensor | None = None,
                frequency_penalties: torch.Tensor | None = None, history: torch.Tensor | None = None,
                uniforms: torch.Tensor | None = None, mass_rows: bool = True) -> torch.Tensor:
        B, V = logits.shape
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        if uniforms is None and not all_greedy:
            uniforms = torch.rand(B, device=logits.device, dtype=torch.float32)
        H = 0 if history is None else int(history.shape[1])
        ws = self.workspace(B, V, logits.dtype, H, logits.device)
        out = torch.empty(B, dtype=torch.int64, device=logits.device)
        sl = lambda t: None if t is None else t[:B].contiguous()
        return sample_into(logits, out, ws, temperatures=None if temperatures is None else sl(temperatures),
                           top_ps=sl(top_ps), top_ks=sl(top_ks), repetition_penalties=sl(repetition_penalties),
                           presence_penalties=sl(presence_penalties), frequency_penalties=sl(frequency_penalties),
                           history=None if history is None else history[:B].contiguous(),
                           uniforms=None if uniforms is None else uniforms[:B].contiguous(),
                           all_greedy=all_greedy, use_top_p=use_top_p, mass_rows=mass_rows)


def argmax_into(logits: torch.Tensor, out_ids: torch.Tensor, workspace: Workspace) -> torch.Tensor:
    """First index of the row maximum (NaN is maximum) into ``out_ids``.

    Replaces ``logits.argmax(-1)`` on the all-greedy path and in the captured
    decode graph (src/compute/model_runner.py:85,353).
    """
    B, V = logits.shape
    if not workspace.fits(B, V, 0):
        raise ValueError("workspace shape mismatch")
    lib = _lib.load()
    _lib.check(lib.qs_argmax(ctypes.c_void_p(logits.data_ptr()), logits.stride(0), _DTYPES[logits.dtype], B, V,
                             ctypes.c_void_p(out_ids.data_ptr()), ctypes.c_void_p(workspace.buf.data_ptr()),
                             workspace.nbytes, ctypes.c_void_p(_stream_handle(logits.device))))
    return out_ids


def sample_gpu(sampler: "BatchSampler", logits: torch.Tensor | list[torch.Tensor], batch) -> torch.Tensor:
    """One token per row: the role of ModelRunner._sample_gpu (src/compute/model_runner.py:77-93).

    ``logits`` is a [B, V] tensor or a list of [1, V] rows (concatenated as at
    model_runner.py:81); ``batch`` is a filled ``SamplingBatch`` whose host flags
    pick the path: all-greedy rows take the argmax kernel (model_runner.py:84-85),
    otherwise the sampler runs with the batch's device buffers (:87-92).
    """
    if isinstance(logits, (list, tuple)):
        if not logits:
            dev = batch.device
            return torch.empty(0, dtype=torch.long, device=dev)
        logits = torch.cat(list(logits), dim=0)
    B, V = logits.shape
    if batch.all_greedy:
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        ws = sampler.workspace(B, V, logits.dtype, 0, logits.device)
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
              uniforms: torch.Tensor, all_greedy: bool, use_top_p: bool) -> torch.Tensor:
    """Custom-op boundary for compiled callers (pattern of src/compute/layers/ops.py:18-39)."""
    return _default_sampler()(logits, temperatures, top_ps, all_greedy=all_greedy, use_top_p=use_top_p,
                              top_ks=top_ks, uniforms=uniforms)


@sample_op.register_fake
def _sample_op_fake(logits, temperatures, top_ps, top_ks, uniforms, all_greedy, use_top_p):
    return torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
