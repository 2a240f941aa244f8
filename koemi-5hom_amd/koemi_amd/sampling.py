"""Decode-step token selection on the GPU: the reference's ``SamplingPolicy``
and ``TokenSampler`` (runtime/fast_decode.py:20-95) on one HIP kernel each.

Greedy selection runs ``koemi_herm_greedy_tokens`` (the padding id masked, the
first maximum winning, as ``argmax`` after ``index_fill`` does). Sampling runs
``koemi_herm_sample_tokens``: the padding id removed, the top-k restriction
(every score below the k-th largest set to -inf, ties kept), ``softmax(scores
/ temperature)``, then an inverse-CDF draw from a uniform number per row that
this front draws with ``torch.rand`` from the sampler's generator (the
reference draws with ``torch.multinomial``; the kernel takes the uniforms as
an input so that a captured decode graph can draw from numbers written into
a static buffer before each replay). Nothing is read back to the host.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from koemi_amd import _native

__all__ = ["PAD_TOKEN_ID", "SamplingPolicy", "TokenSampler"]

PAD_TOKEN_ID = 256  # configuration/settings.py:10-11


@dataclass(frozen=True)
class SamplingPolicy:
    """Token selection rule applied to one decode step (fast_decode.py:20-37).

    ``temperature`` scales the logits and must be positive. ``top_k`` keeps only
    the highest scoring ids before sampling. ``greedy`` takes the argmax and
    ignores both. The padding id is always removed before selection."""

    temperature: float = 1.0
    top_k: int | None = None
    greedy: bool = False

    def __post_init__(self) -> None:
        if self.temperature <= 0.0:
            raise ValueError("temperature must be positive")
        if self.top_k is not None:
            if isinstance(self.top_k, bool) or not isinstance(self.top_k, int) or self.top_k < 1:
                raise ValueError("top_k must be a positive integer")


class TokenSampler:
    """Select decode tokens without reading a tensor value back to the host
    (fast_decode.py:40-95): ``sampler(logits)`` for ``[batch, vocabulary]``
    logits returns ``[batch, 1]`` int64 ids; ``probabilities(logits)`` the
    distribution the policy draws from; ``sample_with_probabilities`` both.
    ``uniforms`` (keyword-only, build-side): ``[batch]`` fp32 numbers in
    [0, 1) to draw with instead of drawing them from ``generator``."""

    def __init__(self, policy: SamplingPolicy, device: torch.device, generator: torch.Generator | None = None) -> None:
        self.policy = policy
        self.device = torch.device(device)
        self.generator = generator

    def _scores(self, logits: Tensor) -> Tensor:
        if logits.ndim != 2:
            raise ValueError("sampling requires logits with shape [batch, vocabulary]")
        if logits.device.type != "cuda":
            raise ValueError("sampling requires CUDA logits")
        scores = logits if logits.dtype == torch.float32 else logits.float()
        return scores if scores.stride(1) == 1 else scores.contiguous()

    def _draw(self, scores: Tensor, probabilities: Tensor | None, uniforms: Tensor | None) -> Tensor:
        batch, vocab = scores.shape
        ids = torch.empty((batch, 1), device=scores.device, dtype=torch.int64)
        if self.policy.greedy:
            _native.call("koemi_herm_greedy_tokens", _native.ptr(scores), scores.stride(0), batch, vocab,
                         PAD_TOKEN_ID, _native.ptr(ids), _native.stream_of(scores.device))
            if probabilities is not None:
                probabilities.zero_().scatter_(-1, ids, 1.0)
            return ids
        if uniforms is None:
            uniforms = torch.rand((batch,), device=scores.device, dtype=torch.float32, generator=self.generator)
        elif uniforms.shape != (batch,) or uniforms.dtype != torch.float32 or uniforms.device != scores.device:
            raise ValueError("uniforms must be a float32 [batch] tensor on the logits' device")
        _native.call("koemi_herm_sample_tokens", _native.ptr(scores), scores.stride(0), batch, vocab, PAD_TOKEN_ID,
                     float(self.policy.temperature), int(self.policy.top_k or 0), _native.ptr(uniforms.contiguous()),
                     _native.ptr(ids), _native.ptr(probabilities), _native.stream_of(scores.device))
        return ids

    def probabilities(self, logits: Tensor) -> Tensor:
        """The distribution this policy draws from, for [batch, vocabulary] logits."""
        return self.sample_with_probabilities(logits)[1]

    def sample_with_probabilities(self, logits: Tensor, *, uniforms: Tensor | None = None) -> tuple[Tensor, Tensor]:
        """[batch, 1] sampled ids together with the distribution they came from."""
        scores = self._scores(logits)
        probabilities = torch.empty(scores.shape, device=scores.device, dtype=torch.float32)
        ids = self._draw(scores, probabilities, uniforms)
        return ids, probabilities

    def __call__(self, logits: Tensor, *, uniforms: Tensor | None = None) -> Tensor:
        """[batch, 1] sampled ids for [batch, vocabulary] logits."""
        return self._draw(self._scores(logits), None, uniforms)
