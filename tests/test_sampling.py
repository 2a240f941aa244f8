"""SamplingPolicy / TokenSampler fronts (runtime/fast_decode.py:20-95): the
reference's validation, with its messages, on the CPU."""

from __future__ import annotations

import pytest
import torch

from koemi_amd.sampling import SamplingPolicy, TokenSampler


@pytest.mark.parametrize("kwargs, message", [
    ({"temperature": 0.0}, "temperature must be positive"),
    ({"temperature": -1.0}, "temperature must be positive"),
    ({"top_k": 0}, "top_k must be a positive integer"),
    ({"top_k": True}, "top_k must be a positive integer"),
    ({"top_k": 2.0}, "top_k must be a positive integer"),
])
def test_policy_rejects_what_the_reference_rejects(kwargs, message):
    with pytest.raises(ValueError, match=message):
        SamplingPolicy(**kwargs)


def test_policy_defaults_and_sampler_shape_check():
    policy = SamplingPolicy()
    assert (policy.temperature, policy.top_k, policy.greedy) == (1.0, None, False)
    sampler = TokenSampler(SamplingPolicy(top_k=3), torch.device("cpu"))
    with pytest.raises(ValueError, match=r"\[batch, vocabulary\]"):
        sampler(torch.zeros((2, 3, 257)))
