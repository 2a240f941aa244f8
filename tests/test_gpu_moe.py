"""GPU parity of the MoE fronts: route, permute, grouped GLU-FFN, combine.

* routing indices, learned top-k indices, expert counts, permutation order,
  sorted rows/experts, segment offsets and sorted context: bit-exact against the
  oracle (C4: T = 32768, D = 1024 bf16, E = 16, k = 2; hash and learned gates);
* learned gate weights: bit-exact against the oracle (same exp and sum order),
  within 1e-6 relative of torch softmax;
* grouped MLP: fp32 path 2e-4 (tests/cuda/test_moe_cuda.py:113); bf16 MFMA path
  against the float64 oracle with the GLU product rounded to bf16 as the kernel
  stores it: |err| <= 2^-7 |y| + 2e-3 max|y| per element (bf16 output rounding
  plus fp32-accumulation order), max abs / rel printed;
* combine: bit-exact against the oracle's ascending-order fp32 sum rounded once.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from koemi_amd import moe, workloads

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "kats.json").read_text())


def bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


# ------------------------------------------------------------------- route


def test_route_matches_reference_test_and_kat(device):
    tok = torch.tensor([[1, 2, 99], [7, 3, 4]], device=device)
    prev = torch.tensor([[0, 1, 2], [6, 7, 8]], device=device)
    valid = torch.tensor([[True, True, False], [True, False, True]], device=device)
    got = moe.route_topk_valid(tok, prev, valid, expert_count=8, top_k=2)
    want = oracle.route_hash(tok.cpu().numpy(), prev.cpu().numpy(), valid.cpu().numpy(), 8, 2)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    kat = GOLDEN["network_hash_route"]
    t = torch.tensor(kat["token_ids"], device=device)
    p = torch.tensor(kat["previous_token_ids"], device=device)
    v = t != 256
    a = moe.route_topk_valid(t, p, v, expert_count=kat["expert_count"], top_k=1)
    assert a[..., 0].tolist() == kat["expert_indices"]
    counts = moe.expert_activation_counts(a, v, expert_count=kat["expert_count"])
    assert counts.tolist() == kat["activation_counts"]


@pytest.mark.parametrize("id_dtype", [torch.int64, torch.int32])
def test_config4_hash_route_bit_exact(device, id_dtype):
    c = workloads.config4()
    got = moe.route_topk_valid(c.token_ids.to(device, id_dtype), c.previous_token_ids.to(device, id_dtype),
                               c.valid.to(device), expert_count=16, top_k=2)
    want = oracle.route_hash(c.token_ids.numpy(), c.previous_token_ids.numpy(), c.valid.numpy(), 16, 2)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    counts = moe.expert_activation_counts(got, c.valid.to(device), expert_count=16)
    np.testing.assert_array_equal(counts.cpu().numpy(), oracle.expert_counts(want, c.valid.numpy(), 16))


@pytest.mark.parametrize("id_dtype", [torch.int64, torch.int32])
def test_config4_modulo_route_bit_exact(device, id_dtype):
    """The C4 synthetic variant "token id mod 16" (slot k -> (tok + k) mod 16):
    assignments, counts and the permutation bit-exact against the oracle, with
    some tokens invalid and, in a second call, negative ids."""

    c = workloads.config4()
    valid = c.valid.clone()
    valid[5::113] = False
    got = moe.route_topk_modulo(c.token_ids.to(device, id_dtype), valid.to(device), expert_count=16, top_k=2)
    want = oracle.route_modulo(c.token_ids.numpy(), valid.numpy(), 16, 2)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    counts = moe.expert_activation_counts(got, valid.to(device), expert_count=16)
    np.testing.assert_array_equal(counts.cpu().numpy(), oracle.expert_counts(want, valid.numpy(), 16))
    sc, rows, experts, offsets = moe.permute_topk(c.context.to(device), got, valid.to(device), expert_count=16)
    w_sc, w_rows, w_experts, w_off = oracle.permute(bf16_np(c.context), want, valid.numpy(), 16)
    np.testing.assert_array_equal(rows.cpu().numpy(), w_rows)
    np.testing.assert_array_equal(experts.cpu().numpy(), w_experts)
    np.testing.assert_array_equal(offsets.cpu().numpy(), w_off)
    np.testing.assert_array_equal(bf16_np(sc), w_sc)
    neg = torch.arange(-40, 40, dtype=id_dtype, device=device)
    ok = torch.ones(80, dtype=torch.bool, device=device)
    np.testing.assert_array_equal(moe.route_topk_modulo(neg, ok, expert_count=7, top_k=3).cpu().numpy(),
                                  oracle.route_modulo(neg.cpu().numpy(), ok.cpu().numpy(), 7, 3))


def test_route_rejects_duplicate_slots(device):
    tok = torch.arange(64, device=device)
    with pytest.raises(moe.CudaMoeValidationError, match="duplicate experts"):
        moe.route_topk_valid(tok, tok, torch.ones(64, dtype=torch.bool, device=device), expert_count=3, top_k=2)


def test_config4_learned_route_bit_exact(device):
    c = workloads.config4()
    valid = c.valid.clone()
    valid[::97] = False
    idx, w = moe.route_topk_learned(c.router_logits.to(device), valid.to(device), top_k=2)
    want_idx, want_w = oracle.route_learned(c.router_logits.numpy(), valid.numpy(), 2)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_array_equal(w.cpu().numpy(), want_w)
    ref_w, ref_idx = c.router_logits.softmax(-1).topk(2, dim=-1)
    v = valid.numpy()
    np.testing.assert_array_equal(idx.cpu().numpy()[v], ref_idx.numpy()[v])
    np.testing.assert_allclose(w.cpu().numpy()[v], ref_w.numpy()[v], rtol=1e-6)


def _check_router_statistics(stats, want, tokens):
    """RouterStatistics on the device against the float64 oracle. The mass is
    an fp32 sum of positive terms, 256 tokens per workgroup in order, then
    the workgroups in order, each term within 4 ulp (fixed exp, one division):
    relative error <= (256 + workgroups + 4) * 2^-24 per expert; counts and the
    valid count are exact integers; the loss adds its own fp32 steps."""
    u = 2.0 ** -24
    rel = (256 + (tokens + 255) // 256 + 4) * u
    mass = stats.probability_mass.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(mass - want["probability_mass"]) <= rel * want["probability_mass"] + 1e-30), \
        f"mass err {np.abs(mass - want['probability_mass']).max():.3e}"
    np.testing.assert_array_equal(stats.assignment_counts.cpu().numpy(), want["assignment_counts"])
    assert float(stats.valid_count) == want["valid_count"]
    assert stats.valid_count.shape == () and stats.balance_loss.shape == ()
    loss = float(stats.balance_loss)
    E = mass.size
    assert abs(loss - want["balance_loss"]) <= (rel + (2 * E + 8) * u) * max(want["balance_loss"], 1e-30), \
        f"loss {loss!r} vs {want['balance_loss']!r}"


def test_config4_router_statistics(device):
    """LearnedExpertMixture.forward's statistics at C4 (router.py:50-58): the
    route's bits equal the plain learned route's, the statistics match the
    float64 oracle, and the balance loss formed by the standalone kernel from
    the same statistics equals the fused one bit for bit."""
    c = workloads.config4()
    valid = c.valid.clone()
    valid[::97] = False
    logits = c.router_logits.to(device)
    idx, w, stats = moe.route_topk_learned(logits, valid.to(device), top_k=2, return_statistics=True)
    idx0, w0 = moe.route_topk_learned(logits, valid.to(device), top_k=2)
    assert torch.equal(idx, idx0) and torch.equal(w, w0)
    want = oracle.router_statistics(c.router_logits.numpy(), valid.numpy(), idx.cpu().numpy())
    _check_router_statistics(stats, want, c.router_logits.shape[0])
    again = moe.RouterStatistics(stats.probability_mass, stats.assignment_counts, stats.valid_count)
    assert torch.equal(again.balance_loss, stats.balance_loss)
    # deterministic: a second call gives the same bits
    _, _, stats2 = moe.route_topk_learned(logits, valid.to(device), top_k=2, return_statistics=True)
    assert torch.equal(stats2.probability_mass, stats.probability_mass)


@pytest.mark.parametrize("tokens, experts, k", [(1000, 100, 3), (257, 4, 2), (5, 1024, 8), (3000, 16, 1)])
def test_router_statistics_shapes(device, tokens, experts, k):
    """A last workgroup of a few tokens, experts beyond one 64-expert chunk
    (100: two chunks, 1024: sixteen), k from 1 to 8, a fifth of the tokens
    invalid."""
    g = torch.Generator().manual_seed(tokens + experts)
    logits = 2.0 * torch.randn((tokens, experts), generator=g)
    valid = torch.rand((tokens,), generator=g) > 0.2
    idx, w, stats = moe.route_topk_learned(logits.to(device), valid.to(device), top_k=k, return_statistics=True)
    want_idx, want_w = oracle.route_learned(logits.numpy(), valid.numpy(), k)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_array_equal(w.cpu().numpy(), want_w)
    _check_router_statistics(stats, oracle.router_statistics(logits.numpy(), valid.numpy(), want_idx), tokens)


def test_router_statistics_empty_and_merged(device):
    """An empty mask gives zero statistics and a zero loss
    (test_learned_router.py:82-87); no tokens at all as well; statistics of
    two halves merged (router.py:25-32) match the oracle's merge, their loss
    formed on the device."""
    g = torch.Generator().manual_seed(5)
    logits = torch.randn((600, 16), generator=g)
    none = torch.zeros((600,), dtype=torch.bool)
    _, _, stats = moe.route_topk_learned(logits.to(device), none.to(device), top_k=2, return_statistics=True)
    assert float(stats.valid_count) == 0 and float(stats.balance_loss) == 0.0
    assert not stats.probability_mass.any() and not stats.assignment_counts.any()
    idx, _, stats = moe.route_topk_learned(logits[:0].to(device), none[:0].to(device), top_k=2,
                                           return_statistics=True)
    assert idx.shape == (0, 2) and float(stats.valid_count) == 0 and float(stats.balance_loss) == 0.0
    valid = torch.rand((600,), generator=g) > 0.3
    halves = [moe.route_topk_learned(logits[s].to(device), valid[s].to(device), top_k=2, return_statistics=True)
              for s in (slice(0, 300), slice(300, 600))]
    merged = moe.merge_router_statistics([h[2] for h in halves])
    want = oracle.merge_router_statistics([
        oracle.router_statistics(logits[s].numpy(), valid[s].numpy(), h[0].cpu().numpy())
        for s, h in zip((slice(0, 300), slice(300, 600)), halves)])
    _check_router_statistics(merged, want, 600)
    assert moe.merge_router_statistics([]) is None


# ----------------------------------------------------------------- permute


def test_permute_known_answer(device):
    kat = GOLDEN["permute_stable_pairs"]
    ctx = torch.arange(kat["context_rows"] * kat["context_width"], dtype=torch.float32).reshape(kat["context_rows"], -1)
    sc, rows, experts, offsets = moe.permute_topk(ctx.to(device), torch.tensor(kat["assignments"], device=device),
                                                  torch.tensor(kat["valid"], device=device), expert_count=kat["expert_count"])
    assert rows.tolist() == kat["sorted_rows"] and experts.tolist() == kat["sorted_experts"]
    assert offsets.tolist() == kat["segment_offsets"]
    z = kat["zero_rows_from"]
    assert torch.equal(sc[:z].cpu(), ctx[torch.tensor(kat["sorted_rows"][:z])])
    assert torch.equal(sc[z:].cpu(), torch.zeros_like(sc[z:].cpu()))
    outputs = sc + 10.0
    combined = moe.combine_topk(outputs, rows, offsets, token_count=3, top_k=2)
    expected = torch.zeros_like(ctx)
    for pair in range(kat["segment_offsets"][-1]):
        expected[rows[pair].item()] += outputs[pair].cpu() / 2.0
    assert torch.equal(combined.cpu(), expected)


@pytest.mark.parametrize(
    "dtype, T, k, E",
    [(torch.float32, 5000, 3, 13), (torch.bfloat16, 5000, 3, 13), (torch.float16, 5000, 3, 13),
     # count tables too large to stage in LDS (and E + 1 > 1024): the global-memory scan
     (torch.bfloat16, 3000, 2, 1500), (torch.float32, 40000, 2, 24),
     # at most 1024 pairs and 64 keys: the one-workgroup index phase (a decode step: 64 tokens x top-2)
     (torch.bfloat16, 64, 2, 16), (torch.float32, 341, 3, 13), (torch.float16, 1024, 1, 63), (torch.float32, 1, 2, 2),
     (torch.bfloat16, 512, 2, 64)],
)
def test_permute_random_with_invalid_and_repeats(device, dtype, T, k, E):
    g = torch.Generator().manual_seed(71)
    D = 72
    a = torch.randint(-1, E + 1, (T, k), generator=g)
    valid = torch.rand((T,), generator=g) > 0.2
    ctx = torch.randn((T, D), generator=g).to(dtype)
    w = torch.rand((T, k), generator=g)
    got = moe.permute_topk(ctx.to(device), a.to(device), valid.to(device), expert_count=E, pair_weights=w.to(device), validate=False)
    want = oracle.permute(ctx.float().numpy(), a.numpy(), valid.numpy(), E, pair_weights=w.numpy())
    np.testing.assert_array_equal(got[0].float().cpu().numpy(), want[0])
    for g_t, w_t in zip(got[1:], want[1:]):
        np.testing.assert_array_equal(g_t.cpu().numpy(), w_t)


def test_config4_permute_bit_exact(device):
    c = workloads.config4()
    a = oracle.route_hash(c.token_ids.numpy(), c.previous_token_ids.numpy(), c.valid.numpy(), 16, 2)
    got = moe.permute_topk(c.context.to(device), torch.from_numpy(a).to(device), c.valid.to(device), expert_count=16)
    want = oracle.permute(c.context.view(torch.int16).numpy(), a, c.valid.numpy(), 16)
    assert torch.equal(got[0].view(torch.int16).cpu(), torch.from_numpy(want[0]))
    for g_t, w_t in zip(got[1:], want[1:]):
        np.testing.assert_array_equal(g_t.cpu().numpy(), w_t)


# ------------------------------------------------------------- grouped MLP


def test_grouped_mlp_fp32_matches_reference_rows(device):
    torch.manual_seed(3)
    E, D, H, P = 2, 4, 3, 3
    x = torch.randn(P, D, device=device)
    experts = torch.tensor([0, 0, 1], device=device)
    offsets = torch.tensor([0, 2, 3], device=device)
    gw, gb = torch.randn(E, H, D, device=device), torch.randn(E, H, device=device)
    vw, vb = torch.randn_like(gw), torch.randn_like(gb)
    ow, ob = torch.randn(E, D, H, device=device), torch.randn(E, D, device=device)
    got = moe.grouped_expert_mlp_inference(x, experts, offsets, gw, gb, vw, vb, ow, ob)
    rows = []
    for row, e in enumerate(experts.tolist()):
        gate = F.linear(x[row], gw[e], gb[e])
        value = F.linear(x[row], vw[e], vb[e])
        rows.append(F.linear(F.silu(gate) * value, ow[e], ob[e]))
    torch.testing.assert_close(got, torch.stack(rows), rtol=2e-4, atol=2e-4)


def check_bf16_mlp(got: torch.Tensor, want: np.ndarray, name: str):
    g = got.float().cpu().numpy()
    err = np.abs(g - want)
    scale = np.abs(want).max()
    print(f"{name}: max_abs={err.max():.3e} max|y|={scale:.3e} max_rel_to_scale={err.max() / scale:.3e}", flush=True)
    assert np.all(err <= 2.0**-7 * np.abs(want) + 2e-3 * scale)


@pytest.mark.parametrize("sizes", [(0, 5, 300, 0, 57), (128, 128, 1, 255, 3), (1000, 0, 0, 17, 2)])
def test_grouped_mlp_bf16_mfma_ragged_segments(device, sizes):
    g = torch.Generator().manual_seed(sum(sizes))
    E, D, H = len(sizes), 256, 384
    offsets = np.concatenate([[0], np.cumsum(sizes)])
    P = int(offsets[-1]) + 7  # trailing rows past the valid pairs
    x = torch.randn((P, D), generator=g).to(torch.bfloat16)
    experts = torch.full((P,), E, dtype=torch.int64)
    for e in range(E):
        experts[offsets[e]:offsets[e + 1]] = e
    ws = [(0.05 * torch.randn(s, generator=g)).to(torch.bfloat16) for s in ((E, H, D), (E, H), (E, H, D), (E, H), (E, D, H), (E, D))]
    got = moe.grouped_expert_mlp_inference(x.to(device), experts.to(device), torch.from_numpy(offsets).to(device),
                                           *(w.to(device) for w in ws))
    want = oracle.grouped_mlp(x.float().numpy(), experts.numpy(), offsets, *(w.float().numpy() for w in ws),
                              round_hidden_bf16=True)
    check_bf16_mlp(got, want, f"grouped MLP bf16 sizes={sizes}")
    assert torch.equal(got[offsets[-1]:].cpu(), torch.zeros_like(got[offsets[-1]:].cpu()))


@pytest.mark.parametrize("sizes, D, H", [
    ((0, 5, 70, 0, 57), 256, 384),          # empty experts, a 70-row expert (two passes), a partial second block
    ((33, 1, 64, 65), 128, 192),            # 33 rows (one row in the second block), exactly 64, 65
    ((8, 9, 7, 8, 8, 6, 10, 8, 8, 8, 9, 7, 8, 8, 8, 10), 1024, 2048),  # a C5 decode step: 64 tokens x top-2
    ((0, 40, 70, 0, 3, 100, 0, 1), 1024, 2048),  # C5 widths: empty experts, two to four 32-row passes
])
def test_grouped_mlp_bf16_few_rows_per_expert(device, sizes, D, H):
    """At most 64 pairs per expert on average: the skinny kernels (weights
    streamed once, K split over the waves) against the float64 loop."""
    g = torch.Generator().manual_seed(sum(sizes) + D)
    E = len(sizes)
    offsets = np.concatenate([[0], np.cumsum(sizes)])
    P = int(offsets[-1]) + 5  # trailing rows past the valid pairs
    assert P <= 64 * E
    x = torch.randn((P, D), generator=g).to(torch.bfloat16)
    experts = torch.full((P,), E, dtype=torch.int64)
    for e in range(E):
        experts[offsets[e]:offsets[e + 1]] = e
    ws = [(0.05 * torch.randn(s, generator=g)).to(torch.bfloat16) for s in ((E, H, D), (E, H), (E, H, D), (E, H), (E, D, H), (E, D))]
    got = moe.grouped_expert_mlp_inference(x.to(device), experts.to(device), torch.from_numpy(offsets).to(device),
                                           *(w.to(device) for w in ws))
    want = oracle.grouped_mlp(x.float().numpy(), experts.numpy(), offsets, *(w.float().numpy() for w in ws),
                              dtype=np.float32, round_hidden_bf16=True)
    check_bf16_mlp(got[:offsets[-1]], want[:offsets[-1]], f"grouped MLP bf16 skinny sizes={sizes}")
    assert torch.equal(got[offsets[-1]:].cpu(), torch.zeros_like(got[offsets[-1]:].cpu()))


@pytest.mark.parametrize("E", [64, 65, 90])
def test_grouped_mlp_bf16_many_experts(device, E):
    """Many experts, with empty, one-row, whole-tile and ragged segments among
    them: the tile schedule (per-expert tile counts, their prefix, the
    expert of every slot) and the tiles against the float64 loop."""
    g = torch.Generator().manual_seed(E)
    D, H = 128, 192
    sizes = torch.randint(0, 420, (E,), generator=g)
    sizes[::7] = 0
    sizes[3::11] = 1
    sizes[5::13] = 256
    offsets = np.concatenate([[0], np.cumsum(sizes.numpy())])
    P = int(offsets[-1]) + 6
    assert P > 64 * E  # the tiled path
    x = torch.randn((P, D), generator=g).to(torch.bfloat16)
    experts = torch.full((P,), E, dtype=torch.int64)
    for e in range(E):
        experts[offsets[e]:offsets[e + 1]] = e
    ws = [(0.05 * torch.randn(s, generator=g)).to(torch.bfloat16) for s in ((E, H, D), (E, H), (E, H, D), (E, H), (E, D, H), (E, D))]
    got = moe.grouped_expert_mlp_inference(x.to(device), experts.to(device), torch.from_numpy(offsets).to(device),
                                           *(w.to(device) for w in ws))
    want = oracle.grouped_mlp(x.float().numpy(), experts.numpy(), offsets, *(w.float().numpy() for w in ws),
                              dtype=np.float32, round_hidden_bf16=True)
    check_bf16_mlp(got[:offsets[-1]], want[:offsets[-1]], f"grouped MLP bf16 E={E}")
    assert torch.equal(got[offsets[-1]:].cpu(), torch.zeros_like(got[offsets[-1]:].cpu()))


@pytest.mark.parametrize("sizes", [(16640, 16600), (20992, 21208)])
def test_grouped_mlp_bf16_whole_rounds_and_split_last_round(device, sizes):
    # Width 512 and hidden 256 give two tiles per row slot in both GEMMs. On a
    # 256-CU device (other CU counts take other plans): 130 slots, one whole
    # round plus 4 leftover tiles in four K chunks each; 165 slots (the last
    # one partly filled), one whole round plus 74 leftover tiles in three K
    # chunks each; the fixup kernel sums the chunks in order.
    g = torch.Generator().manual_seed(11)
    E, D, H = 2, 512, 256
    offsets = np.concatenate([[0], np.cumsum(sizes)])
    P = int(offsets[-1]) + 3
    x = torch.randn((P, D), generator=g).to(torch.bfloat16)
    experts = torch.full((P,), E, dtype=torch.int64)
    for e in range(E):
        experts[offsets[e]:offsets[e + 1]] = e
    ws = [(0.05 * torch.randn(s, generator=g)).to(torch.bfloat16) for s in ((E, H, D), (E, H), (E, H, D), (E, H), (E, D, H), (E, D))]
    got = moe.grouped_expert_mlp_inference(x.to(device), experts.to(device), torch.from_numpy(offsets).to(device),
                                           *(w.to(device) for w in ws))
    want = oracle.grouped_mlp(x.float().numpy(), experts.numpy(), offsets, *(w.float().numpy() for w in ws),
                              dtype=np.float32, round_hidden_bf16=True)
    check_bf16_mlp(got[:offsets[-1]], want[:offsets[-1]], "grouped MLP bf16 whole rounds + split last round")
    assert torch.equal(got[offsets[-1]:].cpu(), torch.zeros_like(got[offsets[-1]:].cpu()))


def run_config4_pipeline(device, c, learned: bool):
    ctx = c.context.to(device)
    valid = c.valid.to(device)
    if learned:
        a, w = moe.route_topk_learned(c.router_logits.to(device), valid, top_k=2)
        sc, rows, experts, offsets, sw = moe.permute_topk(ctx, a, valid, expert_count=16, pair_weights=w)
    else:
        a = moe.route_topk_valid(c.token_ids.to(device), c.previous_token_ids.to(device), valid, expert_count=16, top_k=2)
        sc, rows, experts, offsets = moe.permute_topk(ctx, a, valid, expert_count=16)
        sw = None
    y = moe.grouped_expert_mlp_inference(sc, experts, offsets, c.gate_weights.to(device), c.gate_biases.to(device),
                                         c.value_weights.to(device), c.value_biases.to(device),
                                         c.output_weights.to(device), c.output_biases.to(device))
    out = moe.combine_topk(y, rows, offsets, token_count=ctx.shape[0], top_k=2, pair_weights=sw)
    return sc, rows, experts, offsets, sw, y, out


@pytest.mark.parametrize("learned", [False, True])
def test_config4_pipeline(device, learned):
    """C4 end to end. The grouped GLU FFN is checked on every one of the
    65,536 pair rows (all 1024 outputs) against the float64 oracle with bf16
    hidden activations, within oracle.grouped_mlp_bound's per-output bound
    (half an output ulp + one hidden-value ulp of independent sign per term +
    an fp32 accumulation term over K = 2816; its docstring gives the model);
    the rows past the valid pairs are zero."""
    c = workloads.config4()
    sc, rows, experts, offsets, sw, y, out = run_config4_pipeline(device, c, learned)
    off = offsets.cpu().numpy()
    ws = [t.float().numpy() for t in (c.gate_weights, c.gate_biases, c.value_weights, c.value_biases, c.output_weights, c.output_biases)]
    want, bound = oracle.grouped_mlp_bound(sc.float().cpu().numpy(), off, *ws)
    got = y.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - want)
    _, ex = np.frexp(want)
    half_ulp = np.ldexp(1.0, ex - 9)
    name = f"C4 grouped MLP ({'learned' if learned else 'hash'})"
    print(f"{name}: all {got.shape[0]} rows: max err {err.max():.3e}, max err / bound {(err / bound).max():.3f}, "
          f"share above half an ulp {(err > half_ulp).mean():.2e}", flush=True)
    assert np.all(err <= bound), f"{name}: {int((err > bound).sum())} outputs beyond the bound"
    assert not got[int(off[-1]):].any()
    # combine bit-exact against the oracle on the kernel's own expert outputs
    want_out = oracle.combine(y.float().cpu().numpy(), rows.cpu().numpy(), off, c.context.shape[0], 2,
                              None if sw is None else sw.cpu().numpy())
    np.testing.assert_array_equal(out.cpu().view(torch.int16).numpy(), oracle.f32_to_bf16(want_out).view(np.int16))


@pytest.mark.parametrize("tokens, E, D, H, seed", [
    (32768, 16, 1024, 2816, 0),  # C4: whole rounds of 256 x 256 tiles and a split-K last round
    (1500, 7, 192, 320, 1),      # ragged segments, partial tiles
    (64, 16, 1024, 2048, 2),     # a C5 decode step: the few-rows-per-expert kernel
])
def test_indexed_grouped_mlp_equals_the_gathered_one(device, tokens, E, D, H, seed):
    """permute_topk(gather=False) + grouped_expert_mlp_indexed (context rows read
    by sorted_rows inside the first GEMM) give the same bits, on the valid
    pairs, as the gathered sorted context through grouped_expert_mlp_inference:
    the same tiles, the same accumulation order, only the operand addresses
    differ."""
    g = torch.Generator(device=device).manual_seed(seed)
    ctx = torch.randn((tokens, D), generator=g, device=device).to(torch.bfloat16)
    ids = torch.randint(0, 256, (tokens,), generator=g, device=device)
    prev = torch.randint(0, 256, (tokens,), generator=g, device=device)
    valid = torch.rand((tokens,), generator=g, device=device) < 0.95
    a = moe.route_topk_valid(ids, prev, valid, expert_count=E, top_k=2, validate=False)
    ws = [(0.05 * torch.randn(shape, generator=g, device=device)).to(torch.bfloat16)
          for shape in ((E, H, D), (E, H), (E, H, D), (E, H), (E, D, H), (E, D))]
    sc, rows, experts, offsets = moe.permute_topk(ctx, a, valid, expert_count=E)
    none, rows2, experts2, offsets2 = moe.permute_topk(ctx, a, valid, expert_count=E, gather=False)
    assert none is None and torch.equal(rows, rows2) and torch.equal(experts, experts2) and torch.equal(offsets, offsets2)
    want = moe.grouped_expert_mlp_inference(sc, experts, offsets, *ws)
    got = moe.grouped_expert_mlp_indexed(ctx, rows2, offsets2, *ws)
    torch.cuda.synchronize()
    n = int(offsets[-1])  # the rows past the valid pairs are not written by the indexed form
    assert torch.equal(got[:n], want[:n])


@pytest.mark.parametrize("E, rows, cols", [(16, 2048, 1024), (16, 1024, 2048), (3, 96, 192), (1, 32, 64)])
def test_weights_to_fragments_order(device, E, rows, cols):
    """koemi_moe_weights_to_fragments against the layout its declaration
    states: the torch permutation of [E, rows / 32, 32 r, cols / 64 k, 2 half,
    4 j, 8] into [E, rows / 32, k, j, half, r, 8], and the stated offset of
    single elements."""
    g = torch.Generator(device=device).manual_seed(rows + cols)
    w = torch.randn((E, rows, cols), generator=g, device=device).to(torch.bfloat16)
    got = moe.weights_to_fragments(w)
    want = w.view(E, rows // 32, 32, cols // 64, 2, 4, 8).permute(0, 1, 3, 5, 4, 2, 6).reshape(E, rows, cols)
    assert torch.equal(got, want)
    flat_w, flat_got = w.view(-1, cols).cpu(), got.view(-1).cpu()
    for row, c in ((0, 0), (1, 8), (31, 33), (rows - 1, cols - 1), (E * rows - 1, 63), (E * rows // 2 + 5, cols // 2 + 17)):
        b, r = divmod(row, 32)
        at = b * 32 * cols + ((c // 64) * 4 + (c % 32) // 8) * 512 + (32 * ((c % 64) // 32) + r) * 8 + c % 8
        assert flat_got[at] == flat_w[row, c], (row, c)


@pytest.mark.parametrize("sizes, D, H", [
    ((8, 9, 7, 8, 8, 6, 10, 8, 8, 8, 9, 7, 8, 8, 8, 10), 1024, 2048),  # a C5 decode step: 64 tokens x top-2
    ((0, 40, 70, 0, 3, 100, 0, 1), 1024, 2048),  # empty experts, two to four 32-row passes
    ((33, 1, 64, 65), 128, 192),                 # a row in a second block, exactly 64, 65
    ((0, 0, 0, 0), 256, 384),                    # no valid pair
])
def test_fragment_grouped_mlp_equals_the_indexed_one(device, sizes, D, H):
    """grouped_expert_mlp_fragments (weights in fragment order) gives the bits
    of grouped_expert_mlp_indexed on the same pairs: the same products in the
    same order, only the weight addresses differ; the row-major skinny path is
    itself checked against the float64 oracle above."""
    g = torch.Generator(device=device).manual_seed(sum(sizes) + H)
    E = len(sizes)
    tokens = 97
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]), dtype=torch.int64, device=device)
    P = int(offsets[-1]) + 3  # rows past the valid pairs, written by neither
    ctx = torch.randn((tokens, D), generator=g, device=device).to(torch.bfloat16)
    rows = torch.randint(0, tokens, (P,), generator=g, device=device)
    ws = [(0.05 * torch.randn(shape, generator=g, device=device)).to(torch.bfloat16)
          for shape in ((E, H, D), (E, H), (E, H, D), (E, H), (E, D, H), (E, D))]
    frags = [moe.weights_to_fragments(ws[i]) for i in (0, 2, 4)]
    want = moe.grouped_expert_mlp_indexed(ctx, rows, offsets, *ws)
    got = moe.grouped_expert_mlp_fragments(ctx, rows, offsets, frags[0], ws[1], frags[1], ws[3], frags[2], ws[5])
    torch.cuda.synchronize()
    n = int(offsets[-1])
    assert torch.equal(got[:n], want[:n])
    with pytest.raises(moe.CudaMoeValidationError):
        moe.grouped_expert_mlp_fragments(ctx, torch.zeros(64 * E + 1, dtype=torch.int64, device=device), offsets,
                                         frags[0], ws[1], frags[1], ws[3], frags[2], ws[5])


@pytest.mark.parametrize("tokens, k, E, id_dtype", [(32768, 2, 16, torch.int64), (64, 2, 16, torch.int64),
                                                     (5000, 3, 13, torch.int32), (1, 2, 4, torch.int64)])
def test_hash_routed_permutation_equals_route_then_permute(device, tokens, k, E, id_dtype):
    """permute_hash_indices (the hash route computed inside the permutation)
    gives the bits of route_topk_valid followed by permute_indices: rows,
    experts, offsets and pair positions, small (one-workgroup) and chunked."""
    g = torch.Generator(device=device).manual_seed(tokens + k)
    ids = torch.randint(-5, 300, (tokens,), generator=g, device=device).to(id_dtype)
    prev = torch.randint(0, 256, (tokens,), generator=g, device=device).to(id_dtype)
    valid = torch.rand((tokens,), generator=g, device=device) < 0.9
    a = moe.route_topk_valid(ids, prev, valid, expert_count=E, top_k=k, validate=False)
    want = moe.permute_indices(a, valid, expert_count=E)
    got = moe.permute_hash_indices(ids, prev, valid, expert_count=E, top_k=k)
    torch.cuda.synchronize()
    for name, w, x in zip(("rows", "experts", "offsets"), want[:3], got[:3]):
        assert torch.equal(w, x), name
    assert torch.equal(want[4], got[4]), "pair positions"


@pytest.mark.parametrize("tokens, k, E, learned", [(64, 2, 16, False), (300, 3, 13, True), (1, 2, 4, False)])
def test_small_combine_bit_exact(device, tokens, k, E, learned):
    """A decode-sized combine (the one-workgroup inversion) against the oracle's
    ascending-order fp32 sums, with and without pair weights."""
    g = torch.Generator().manual_seed(tokens + k)
    D = 96
    a = torch.randint(-1, E + 1, (tokens, k), generator=g)
    valid = torch.rand((tokens,), generator=g) > 0.2
    ctx = torch.randn((tokens, D), generator=g).to(torch.bfloat16)
    w = torch.rand((tokens, k), generator=g) if learned else None
    perm = moe.permute_topk(ctx.to(device), a.to(device), valid.to(device), expert_count=E,
                            pair_weights=w.to(device) if w is not None else None, validate=False)
    sc, rows, offsets = perm[0], perm[1], perm[3]
    sw = perm[4] if w is not None else None
    y = (sc.float() * 1.5 + 0.25).to(torch.bfloat16)  # stand-in expert outputs
    out = moe.combine_topk(y, rows, offsets, token_count=tokens, top_k=k, pair_weights=sw)
    want = oracle.combine(y.float().cpu().numpy(), rows.cpu().numpy(), offsets.cpu().numpy(), tokens, k,
                          pair_weights=sw.cpu().numpy() if sw is not None else None)
    np.testing.assert_array_equal(out.cpu().view(torch.int16).numpy(), oracle.f32_to_bf16(want).view(np.int16))
