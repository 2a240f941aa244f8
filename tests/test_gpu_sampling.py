"""TokenSampler on the GPU (koemi_herm_sample_tokens, koemi_herm_greedy_tokens)
against oracle.sample_tokens (runtime/fast_decode.py:57-95 in float64).

* probabilities within 1e-6 relative + 1e-8 absolute of the oracle's (fp32
  softmax against float64), exactly zero for the PAD column and the columns
  the top-k restriction removes;
* the drawn ids equal the oracle's for the same uniforms wherever the
  uniform is more than 1e-5 from a cumulative boundary (fp32 sums);
* empirical frequencies of 65,536 draws from one row within five standard
  deviations of p;
* the greedy policy equals the masked argmax;
* DecodeGraph with a sampling policy equals eager steps sampled with the
  graph's own uniforms.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from koemi_amd import herm
from koemi_amd.sampling import PAD_TOKEN_ID, SamplingPolicy, TokenSampler

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows, vocab, temperature, top_k", [(64, 257, 1.0, None), (64, 257, 0.8, 40),
                                                             (7, 257, 2.0, 1), (33, 1000, 1.0, 257), (5, 4096, 0.5, 3)])
def test_sampler_matches_the_oracle(device, rows, vocab, temperature, top_k):
    g = torch.Generator().manual_seed(rows + vocab)
    logits = 3.0 * torch.randn((rows, vocab), generator=g)
    logits[0, 5] = logits[0, 6] = 30.0  # a tie at the top
    u = torch.rand((rows,), generator=g)
    sampler = TokenSampler(SamplingPolicy(temperature=temperature, top_k=top_k), device)
    ids, p = sampler.sample_with_probabilities(logits.to(device), uniforms=u.to(device))
    want_ids, want_p = oracle.sample_tokens(logits.numpy(), PAD_TOKEN_ID, temperature, top_k, u.numpy())
    got_p = p.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got_p - want_p) <= 1e-6 * want_p + 1e-8)
    assert np.all(got_p[want_p == 0.0] == 0.0)
    cum = np.cumsum(want_p, axis=1)
    near = np.abs(cum - u.numpy()[:, None]).min(axis=1) <= 1e-5
    got_ids = ids.cpu().numpy()[:, 0]
    np.testing.assert_array_equal(got_ids[~near], want_ids[~near])
    print(f"sampler rows={rows} V={vocab} T={temperature} k={top_k}: near-boundary rows {int(near.sum())}", flush=True)
    again = sampler(logits.to(device), uniforms=u.to(device))
    assert torch.equal(again, ids)


def test_sampler_frequencies_follow_the_probabilities(device):
    n = 65536
    logits = torch.tensor([[2.0, 1.0, 0.5, -1.0, 3.0] + [-30.0] * 252], device=device).repeat(n, 1)
    gen = torch.Generator(device=device).manual_seed(1)
    sampler = TokenSampler(SamplingPolicy(temperature=1.5, top_k=4), device, generator=gen)
    ids, p = sampler.sample_with_probabilities(logits)
    counts = torch.bincount(ids[:, 0], minlength=257).double().cpu()
    prob = p[0].double().cpu()
    assert prob[3] == 0.0 and counts[3] == 0  # fifth largest score: removed by top_k = 4
    sd = torch.sqrt(n * prob * (1 - prob))
    assert bool(((counts - n * prob).abs() <= 5 * sd + 1).all())


def test_greedy_policy_is_the_masked_argmax(device):
    g = torch.Generator().manual_seed(3)
    logits = torch.randn((40, 257), generator=g)
    logits[0, PAD_TOKEN_ID] = 100.0
    ids = TokenSampler(SamplingPolicy(greedy=True), device)(logits.to(device))
    want = logits.index_fill(-1, torch.tensor([PAD_TOKEN_ID]), float("-inf")).argmax(dim=-1, keepdim=True)
    assert torch.equal(ids.cpu(), want)


def test_decode_graph_sampling_equals_eager_steps(device):
    settings = herm.HermSettings(width=64, memory_features=4, local_memory_size=4, salience_memory_size=3,
                                 expert_count=4, top_k=2, layers=2, scan_chunk=8)
    params = herm.prepare_stack(herm.init_stack(settings, 5, device), settings, device)
    b = 8
    ids = torch.randint(0, 256, (b, 1), generator=torch.Generator().manual_seed(2)).to(device)
    policy = SamplingPolicy(temperature=0.9, top_k=20)
    gen = torch.Generator(device=device).manual_seed(9)
    decode = herm.DecodeGraph(params, settings, ids, herm.initial_states(settings, b, device), policy=policy,
                              generator=gen)
    sampler = TokenSampler(policy, device)
    eager_ids, eager_states = ids.clone(), herm.initial_states(settings, b, device)
    for step in range(4):
        logits = decode.run().clone()
        u = decode.uniforms.clone()
        eager_logits, eager_states = herm.stack_window(params, settings, eager_ids, eager_states)
        torch.cuda.synchronize()
        scale = float(eager_logits.abs().max())
        assert float((logits - eager_logits).abs().max()) <= 1e-5 * scale, f"step {step}"
        eager_ids = sampler(eager_logits[:, -1].contiguous(), uniforms=u)
        assert torch.equal(decode.ids, eager_ids), f"step {step}"
