"""Seeded synthetic inputs for the five benchmark configurations.

Every tensor is drawn on the CPU from ``torch.Generator().manual_seed(seed)``
in a fixed order and then copied to the device, so a CPU checker and the GPU
kernels see identical bits. Seeds 1001-1005 name configurations C1-C5.

* C1 affine scan alone: a ~ U(0.80, 0.999), b ~ N(0, 1), [4, 1024, 256] fp32, h0 = 0.
* C2 RMSNorm-SiLU + surprise: x ~ N(0, 1) bf16 [16*2048, 512], gamma ~ 1 + N(0, 0.02)
  bf16 [512], eps 1e-6; logits ~ N(0, 2^2) fp32 [32768, 256]; targets ~ U{0..255};
  all valid; admission above the 0.9 quantile.
* C3 HERM state update at prefill: a = sigmoid(N(2, 1)), b ~ N(0, 0.5^2) fp32
  [32, 4096, 1024], h0 = 0, chunk 64; then RMSNorm-SiLU of h in bf16 with
  gamma ~ 1 + N(0, 0.02) [1024].
* C4 MoE dispatch + experts: ctx ~ N(0, 1) bf16 [32768, 1024]; router logits
  ~ N(0, 1) fp32 [32768, 16]; W_g, W_v ~ N(0, 0.02^2) bf16 [16, 2816, 1024];
  W_o ~ N(0, 0.02^2) bf16 [16, 1024, 2816]; biases ~ N(0, 0.02^2); top-2.
  Hash variant: tok ~ U{0..255}, prev = tok shifted by one with PAD (256) first.
* C5 HERM stack end to end: prefill ids ~ U{0..255} [8, 2048], decode ids
  ~ U{0..255} [64, 1].
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

PAD_TOKEN_ID = 256


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


@dataclass
class ScanInputs:
    retention: torch.Tensor
    increment: torch.Tensor
    initial: torch.Tensor


def config1(scale: int = 1) -> ScanInputs:
    g = _gen(1001)
    shape = (4, 1024 // scale, 256)
    a = torch.rand(shape, generator=g) * (0.999 - 0.80) + 0.80
    b = torch.randn(shape, generator=g)
    return ScanInputs(a, b, torch.zeros((shape[0], shape[2])))


@dataclass
class NormSurpriseInputs:
    x: torch.Tensor        # bf16 [rows, 512]
    gamma: torch.Tensor    # bf16 [512]
    logits: torch.Tensor   # fp32 [rows, 256]
    targets: torch.Tensor  # int64 [rows]
    valid: torch.Tensor    # bool [rows]
    eps: float = 1e-6
    quantile: float = 0.9


def config2(rows: int = 16 * 2048, seed: int = 1002) -> NormSurpriseInputs:
    g = _gen(seed)
    x = torch.randn((rows, 512), generator=g).to(torch.bfloat16)
    gamma = (1.0 + 0.02 * torch.randn((512,), generator=g)).to(torch.bfloat16)
    logits = 2.0 * torch.randn((rows, 256), generator=g)
    targets = torch.randint(0, 256, (rows,), generator=g, dtype=torch.int64)
    valid = torch.ones((rows,), dtype=torch.bool)
    return NormSurpriseInputs(x, gamma, logits, targets, valid)


@dataclass
class StateUpdateInputs:
    retention: torch.Tensor
    increment: torch.Tensor
    initial: torch.Tensor
    gamma: torch.Tensor
    chunk: int = 64
    eps: float = 1e-6


def config3(batch: int = 32, seq: int = 4096, width: int = 1024, seed: int = 1003) -> StateUpdateInputs:
    g = _gen(seed)
    a = torch.sigmoid(torch.randn((batch, seq, width), generator=g) + 2.0)
    b = 0.5 * torch.randn((batch, seq, width), generator=g)
    gamma = (1.0 + 0.02 * torch.randn((width,), generator=g)).to(torch.bfloat16)
    return StateUpdateInputs(a, b, torch.zeros((batch, width)), gamma)


@dataclass
class MoeInputs:
    context: torch.Tensor        # bf16 [T, D]
    router_logits: torch.Tensor  # fp32 [T, E]
    gate_weights: torch.Tensor   # bf16 [E, H, D]
    gate_biases: torch.Tensor    # bf16 [E, H]
    value_weights: torch.Tensor
    value_biases: torch.Tensor
    output_weights: torch.Tensor  # bf16 [E, D, H]
    output_biases: torch.Tensor   # bf16 [E, D]
    token_ids: torch.Tensor       # int64 [T]
    previous_token_ids: torch.Tensor
    valid: torch.Tensor
    top_k: int = 2

    @property
    def expert_count(self) -> int:
        return int(self.gate_weights.shape[0])


def config4(tokens: int = 32768, width: int = 1024, hidden: int = 2816, experts: int = 16, seed: int = 1004,
            weight_dtype: torch.dtype = torch.bfloat16) -> MoeInputs:
    g = _gen(seed)
    ctx = torch.randn((tokens, width), generator=g).to(weight_dtype)
    router = torch.randn((tokens, experts), generator=g)

    def w(*shape: int) -> torch.Tensor:
        return (0.02 * torch.randn(shape, generator=g)).to(weight_dtype)

    gate_w, value_w = w(experts, hidden, width), w(experts, hidden, width)
    out_w = w(experts, width, hidden)
    gate_b, value_b, out_b = w(experts, hidden), w(experts, hidden), w(experts, width)
    tok = torch.randint(0, 256, (tokens,), generator=g, dtype=torch.int64)
    prev = torch.cat((torch.tensor([PAD_TOKEN_ID], dtype=torch.int64), tok[:-1]))
    valid = torch.ones((tokens,), dtype=torch.bool)
    return MoeInputs(ctx, router, gate_w, gate_b, value_w, value_b, out_w, out_b, tok, prev, valid)


def to_device(obj, device: torch.device | str):
    """Copy every tensor field of a workload dataclass to `device`."""

    fields = {name: getattr(obj, name) for name in obj.__dataclass_fields__}
    moved = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in fields.items()}
    return type(obj)(**moved)


@dataclass
class StackInputs:
    prefill_ids: torch.Tensor  # int64 [8, 2048], U{0..255}
    decode_ids: torch.Tensor   # int64 [64, 1], the first decode step's ids


def config5(seed: int = 1005) -> StackInputs:
    """C5 end-to-end: 8 x 2048 prefill byte ids, then greedy decode at batch 64
    from 64 random first ids (the stack's weights: ``herm.init_stack(settings, seed)``)."""

    g = _gen(seed)
    prefill = torch.randint(0, 256, (8, 2048), generator=g, dtype=torch.int64)
    decode = torch.randint(0, 256, (64, 1), generator=g, dtype=torch.int64)
    return StackInputs(prefill, decode)
