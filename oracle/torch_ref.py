"""Torch-CPU restatement of the reference sampler's op sequence -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this module: as the reference-semantics checker, and as the timed CPU
baseline.  The product path (qedge_amd/) never does.

``reference_forward`` follows BatchSampler.forward (src/compute/sampler.py:25-41)
operation for operation on CPU tensors: greedy mask ``T <= 1e-5`` (:30), safe
temperature (:31), fp32 cast, true division and softmax (:32), and, when the
batch uses top-p (:34), a descending sort (:35), the exclusive-prefix-mass mask
``cumsum - p > top_p`` (:36), the masked fill (:37) and ``torch.multinomial``
(:38, :40); greedy rows take ``argmax`` of the raw logits (:41).  The sort is
asked to be stable, which fixes the tie order to ascending token id -- the order
torch's CPU sort gives in practice and the order the kernels use.

``filter_rows`` returns the intermediate state that the drop-in must reproduce
(the surviving set in token-id order, the renormalised post-filter
probabilities, and each token's exclusive prefix mass), so that tests can check
the kernels' sets and probabilities against the reference's own arithmetic.

``extended_forward`` adds the build's extensions in torch ops, in the order the
kernels apply them: history penalties (repetition, then frequency, then
presence), temperature, top-k keeping ties at the k-th value, min_p (keep
p >= min_p * p_max), then top-p on the remaining set.  It is what the CPU baseline times for workloads that use them.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

GREEDY_EPS = 1e-5  # src/compute/sampler.py:30, src/compute/model_runner.py:82


def reference_forward(logits: torch.Tensor, temperatures: torch.Tensor, top_ps: torch.Tensor, *,
                      all_greedy: bool = False, use_top_p: bool = False,
                      generator: torch.Generator | None = None) -> torch.Tensor:
    """BatchSampler.forward (src/compute/sampler.py:25-41) on CPU tensors."""
    if all_greedy:  # :28-29
        return logits.argmax(dim=-1)
    is_greedy = temperatures <= GREEDY_EPS
    divisor = torch.where(is_greedy, torch.ones_like(temperatures), temperatures)
    probs = torch.softmax(logits.float() / divisor.unsqueeze(1), dim=-1)
    if use_top_p:
        desc, order = torch.sort(probs, dim=-1, descending=True, stable=True)
        drop = (desc.cumsum(dim=-1) - desc) > top_ps.unsqueeze(1)
        desc = desc.masked_fill(drop, 0.0)
        drawn = order.gather(1, torch.multinomial(desc, 1, generator=generator)).squeeze(1)
    else:
        drawn = torch.multinomial(probs, 1, generator=generator).squeeze(1)
    return torch.where(is_greedy, logits.argmax(dim=-1), drawn)


def apply_penalties(z: torch.Tensor, history: torch.Tensor, rep: torch.Tensor, pres: torch.Tensor,
                    freq: torch.Tensor) -> torch.Tensor:
    """History penalties on fp32 logits [B, V] (in place on a copy).

    Tokens with history count c > 0: z / rep if z > 0 else z * rep, then
    z - freq * c, then z - pres.  History ids outside [0, V) are padding.
    """
    B, V = z.shape
    out = z.clone()
    valid = (history >= 0) & (history < V)
    counts = torch.zeros((B, V + 1), dtype=torch.int32)
    idx = torch.where(valid, history.long(), torch.full_like(history, V, dtype=torch.long))
    counts.scatter_add_(1, idx, torch.ones_like(idx, dtype=torch.int32))
    counts = counts[:, :V]
    seen = counts > 0
    scaled = torch.where(out > 0, out / rep.unsqueeze(1), out * rep.unsqueeze(1))
    out = torch.where(seen, scaled, out)
    out = torch.where(seen, out - freq.unsqueeze(1) * counts.float(), out)
    out = torch.where(seen, out - pres.unsqueeze(1), out)
    return out


@dataclass
class FilterState:
    z: torch.Tensor          # fp32 [B, V] penalised logits
    probs: torch.Tensor      # fp32 [B, V] softmax of z / T (over the top-k set when top-k is on)
    kept: torch.Tensor       # bool [B, V] surviving set, in token-id order
    post: torch.Tensor       # fp32 [B, V] renormalised post-filter probabilities
    excl: torch.Tensor       # fp32 [B, V] exclusive prefix mass in sorted order, scattered to ids
    greedy: torch.Tensor     # bool [B]
    argmax: torch.Tensor     # int64 [B] argmax of z (first index, NaN is maximum)


def _min_p_mask(scaled: torch.Tensor, min_ps: torch.Tensor) -> torch.Tensor:
    """Tokens with p >= min_p * p_max, evaluated as q - q_max >= log(min_p)."""
    ratio = torch.exp(scaled - scaled.max(dim=-1, keepdim=True).values)
    return ratio >= min_ps.unsqueeze(1)


def filter_rows(logits: torch.Tensor, temperatures: torch.Tensor, top_ps: torch.Tensor | None = None,
                top_ks: torch.Tensor | None = None, rep=None, pres=None, freq=None, history=None,
                use_top_p: bool = True, min_ps: torch.Tensor | None = None) -> FilterState:
    """The reference's filtering state (src/compute/sampler.py:30-37), with the extensions.

    Without penalties and top-k this is exactly the reference's arithmetic; the
    extensions run in the order penalties -> temperature -> top-k -> top-p.
    """
    z = logits.float()
    B, V = z.shape
    if history is not None:
        ones = torch.ones(B)
        z = apply_penalties(z, history, ones if rep is None else rep, 0 * ones if pres is None else pres,
                            0 * ones if freq is None else freq)
    is_greedy = temperatures <= GREEDY_EPS
    divisor = torch.where(is_greedy, torch.ones_like(temperatures), temperatures)
    scaled = z / divisor.unsqueeze(1)
    if top_ks is not None:
        # top-k on the temperature-scaled logits, ties at the k-th value kept
        k = top_ks.long()
        on = (k > 0) & (k < V)
        kk = torch.where(on, k, torch.full_like(k, V))
        kth = torch.sort(scaled, dim=-1, descending=True).values.gather(1, (kk - 1).clamp(min=0).unsqueeze(1))
        scaled = torch.where(on.unsqueeze(1) & (scaled < kth), torch.full_like(scaled, float("-inf")), scaled)
    if min_ps is not None:
        scaled = torch.where(_min_p_mask(scaled, min_ps), scaled, torch.full_like(scaled, float("-inf")))
    probs = torch.softmax(scaled, dim=-1)
    desc, order = torch.sort(probs, dim=-1, descending=True, stable=True)
    excl_sorted = desc.cumsum(dim=-1) - desc
    excl = torch.empty_like(excl_sorted).scatter_(1, order, excl_sorted)
    if use_top_p and top_ps is not None:
        kept = ~(excl > top_ps.unsqueeze(1))
    else:
        kept = torch.ones_like(probs, dtype=torch.bool)
    kept &= probs > 0
    masked = probs.masked_fill(~kept, 0.0)
    post = masked / masked.sum(dim=-1, keepdim=True)
    return FilterState(z, probs, kept, post, excl, is_greedy, logits.argmax(dim=-1))


def extended_forward(logits: torch.Tensor, temperatures: torch.Tensor, top_ps: torch.Tensor | None,
                     top_ks: torch.Tensor | None = None, rep=None, pres=None, freq=None, history=None,
                     use_top_p: bool = True, generator: torch.Generator | None = None,
                     min_ps: torch.Tensor | None = None) -> torch.Tensor:
    """The full extended sampler in torch-CPU ops (penalties, top-k, min_p, top-p, multinomial)."""
    z = logits.float()
    B, V = z.shape
    if history is not None:
        ones = torch.ones(B)
        z = apply_penalties(z, history, ones if rep is None else rep, 0 * ones if pres is None else pres,
                            0 * ones if freq is None else freq)
    is_greedy = temperatures <= GREEDY_EPS
    divisor = torch.where(is_greedy, torch.ones_like(temperatures), temperatures)
    desc_z, order = torch.sort(z / divisor.unsqueeze(1), dim=-1, descending=True, stable=True)
    if top_ks is not None:
        k = top_ks.long()
        on = (k > 0) & (k < V)
        kk = torch.where(on, k, torch.full_like(k, V))
        kth = desc_z.gather(1, (kk - 1).clamp(min=0).unsqueeze(1))
        desc_z = torch.where(desc_z < kth, torch.full_like(desc_z, float("-inf")), desc_z)
    if min_ps is not None:
        desc_z = torch.where(_min_p_mask(desc_z, min_ps), desc_z, torch.full_like(desc_z, float("-inf")))
    desc = torch.softmax(desc_z, dim=-1)
    if use_top_p and top_ps is not None:
        drop = (desc.cumsum(dim=-1) - desc) > top_ps.unsqueeze(1)
        desc = desc.masked_fill(drop, 0.0)
    drawn = order.gather(1, torch.multinomial(desc, 1, generator=generator)).squeeze(1)
    return torch.where(is_greedy, z.argmax(dim=-1), drawn)
