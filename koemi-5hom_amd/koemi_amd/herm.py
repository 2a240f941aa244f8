"""HERM block window and block stack on the GPU (the end-to-end configuration).

``block_window`` is ``KoemiModel.forward_window`` (reference model/network.py:
296-441) under the ablation the reference runs by default, ``no_refine`` (the
memory value is the fast associative read), with hash expert routing (the
static dispatch, experts.py:109-150) or learned routing
(``HermSettings.expert_routing = "learned"``: LearnedExpertMixture,
router.py:43-97) and static rings (``KoemiState.create_static``,
state.py:43-76). Reference checkpoints and ``KoemiState`` map onto this
layout through ``koemi_amd.checkpoint``. Its hot-path operators run on
this package's HIP kernels:

* gates + masking + scan: one stacked GEMM for the two gate projections,
  then ``recurrent.gated_scan`` (memory.py:22-26, network.py:306-310), which
  forms the gates inside the scan kernel;
* surprise from the prior states: ``think.causal_surprise`` on the content
  head (network.py:677-698);
* admission: ``think.salience_admission`` with the fixed threshold (network.py:349);
* local read: ``memory.read_local_window`` (memory.py:332-383);
* salient read: ``memory.read_salient_window`` (memory.py:405-429);
* ring updates: ``window_rings`` (LocalKeyValueMemory.tail and salient_tail,
  memory.py:385-403, 431-455); the reads and the rings take the local keys
  and values in place from the projection, the rings zeroing the entries
  of invalid positions (network.py:337-340) on the way;
* experts: ``moe.route_topk_valid`` (hash) or the gate GEMM then
  ``moe.route_topk_learned`` (learned), ``moe.permute_topk``,
  ``moe.grouped_expert_mlp_inference``, ``moe.combine_topk`` (with the pair
  weights when learned) (experts.py:109-150, 283-289; router.py:43-97;
  layers.py:19-29).

The projections are plain library GEMMs (``torch.nn.functional.linear`` on
hipBLASLt) in ``HermSettings.linear_dtype`` with fp32 results; every other
operation (the associative memory's feature projection included), the
recurrent state and the memories are fp32. bf16 matches the
reference's default GPU precision (``resolve_precision("auto")`` selects bf16
autocast on CUDA, model/gpu_precision.py:96-121); fp32 is the parity setting.
The gate projections are one of those GEMMs (retention and candidate
stacked); their nonlinearity, the mask and the scan run in fp32. The associative memory
(projection tail, write terms, scan-and-read; memory.py:82-144) runs on
``koemi_assoc_scan_read``; the remaining small elementwise steps are torch
operations on device. The local read's novelty output, which only the refine
path reads, is not computed.

The stack (``stack_window``) is this package's composition for the 12-layer
configuration (the reference model is a single block): layer 0 embeds the
token ids, layer l > 0 takes layer l - 1's final context in place of the
embedding (its own input normalizer applied); each layer has its own weights
and state and uses the token ids for validity, routing and surprise targets;
the last layer's head gives the logits. Inference only.
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass
from typing import NamedTuple

import torch
from torch import Tensor
from torch.nn import functional

from koemi_amd import _native, linear, memory, moe, recurrent, think

__all__ = [
    "DecodeGraph",
    "HermSettings",
    "PAD_TOKEN_ID",
    "block_window",
    "SequencePrefill",
    "WavefrontPrefill",
    "WindowGraph",
    "associative_scan_read",
    "associative_scan_read_windows",
    "block_sequence",
    "stack_sequence",
    "window_rings",
    "decode_step",
    "init_stack",
    "initial_states",
    "prefill",
    "prefill_graphed",
    "prepare_stack",
    "stack_window",
]

PAD_TOKEN_ID = 256             # configuration/settings.py:10-11
_EPS = 1e-6                    # RootMeanSquareNorm epsilon (layers.py:9)


@dataclass(frozen=True)
class HermSettings:
    """Model settings (configuration/settings.py:14-32 names) of the stack."""

    width: int = 1024
    memory_features: int = 16
    local_memory_size: int = 16
    salience_memory_size: int = 16
    salience_threshold: float = 0.75
    expert_count: int = 16
    top_k: int = 2
    vocabulary_size: int = PAD_TOKEN_ID + 1
    layers: int = 12
    scan_chunk: int = 128
    linear_dtype: torch.dtype = torch.bfloat16
    expert_routing: str = "hash"   # "hash" (experts.py:109-150) or "learned" (router.py:43-97)
    ablation: str = "no_refine"    # "no_refine" (the default) or "herm" (the refine memory, network.py:359-384)
    refine_decay_rate: float = 0.0625  # configuration/settings.py:29

    def __post_init__(self) -> None:
        if self.ablation not in ("no_refine", "herm"):
            raise ValueError(f"ablation must be no_refine or herm, not {self.ablation!r}")
        if not 0.0 < self.refine_decay_rate <= 1.0:
            raise ValueError("refine_decay_rate must be greater than zero and at most one")

    @property
    def refine(self) -> bool:
        return self.ablation == "herm"

    def oracle_config(self) -> dict:
        keys = ("width", "memory_features", "local_memory_size", "salience_memory_size", "salience_threshold",
                "expert_count", "top_k", "expert_routing", "ablation", "refine_decay_rate")
        values = asdict(self)
        return {k: values[k] for k in keys}


def _linear_init(generator: torch.Generator, out_features: int, in_features: int) -> tuple[Tensor, Tensor]:
    """nn.Linear's default initialisation: U(-1/sqrt(in), 1/sqrt(in)) for weight and bias."""

    bound = 1.0 / math.sqrt(in_features)
    device = generator.device
    weight = (torch.rand((out_features, in_features), generator=generator, device=device) * 2.0 - 1.0) * bound
    bias = (torch.rand((out_features,), generator=generator, device=device) * 2.0 - 1.0) * bound
    return weight, bias


def init_stack(settings: HermSettings, seed: int, device: torch.device | str = "cpu") -> list[dict[str, Tensor]]:
    """Random-initialised fp32 parameters of every layer, from one seeded
    generator on ``device`` (nn.Embedding ~ N(0, 1) with the padding row zero,
    nn.Linear uniform, normalizer weights one; network.py:81-106)."""

    g = torch.Generator(device=device).manual_seed(seed)
    d, m, e, v = settings.width, settings.memory_features, settings.expert_count, settings.vocabulary_size
    hidden = 2 * d  # GatedFeedForward expands to 2 x width (layers.py:22)
    layers = []
    for layer in range(settings.layers):
        p: dict[str, Tensor] = {}
        if layer == 0:
            p["embedding"] = torch.randn((v, d), generator=g, device=device)
            p["embedding"][PAD_TOKEN_ID] = 0.0
        p["input_norm"] = torch.ones(d, device=device)
        for name in ("retention", "candidate", "key", "query", "value", "local_key", "local_value"):
            p[name + "_w"], p[name + "_b"] = _linear_init(g, d, d)
        p["feature_w"], p["feature_b"] = _linear_init(g, m, d)
        p["decay_w"], p["decay_b"] = _linear_init(g, 1, d)
        p["write_w"], p["write_b"] = _linear_init(g, 1, d)
        p["fusion_w"], p["fusion_b"] = _linear_init(g, d, 4 * d)
        p["fusion_norm"] = torch.ones(d, device=device)
        for name, (o, i) in (("gate", (hidden, d)), ("up", (hidden, d)), ("down", (d, hidden))):
            pairs = [_linear_init(g, o, i) for _ in range(e)]
            p[name + "_w"] = torch.stack([w for w, _ in pairs])
            p[name + "_b"] = torch.stack([b for _, b in pairs])
        p["expert_norm"] = torch.ones(d, device=device)
        if settings.expert_routing == "learned":
            bound = 1.0 / math.sqrt(d)  # nn.Linear(d, E, bias=False) (router.py:41)
            p["router_w"] = (torch.rand((e, d), generator=g, device=device) * 2.0 - 1.0) * bound
        p["head_w"], p["head_b"] = _linear_init(g, v, d)
        if settings.refine:  # memory_refine_gate = nn.Linear(4 width, 1) (network.py:94-96)
            p["refine_gate_w"], p["refine_gate_b"] = _linear_init(g, 1, 4 * d)
        layers.append(p)
    return layers


def prepare_stack(params: list[dict[str, Tensor]], settings: HermSettings, device: torch.device) -> list[dict[str, Tensor]]:
    """Device copies laid out for the kernels: the projections of the working
    states stacked into one GEMM (local key, local value, value, the key's and
    the query's feature logits with W_f folded in, decay, write), the two gate
    projections stacked into another, the GEMM weights in ``linear_dtype``
    with fp32 biases, the content head in fp32."""

    lin = settings.linear_dtype
    prepared = []
    for p in params:
        q: dict[str, Tensor] = {}
        to = lambda t, dtype=torch.float32: t.to(device=device, dtype=dtype).contiguous()
        if "embedding" in p:
            q["embedding"] = to(p["embedding"])
        q["input_norm"] = to(p["input_norm"])
        q["gates_w"] = to(torch.cat((p["retention_w"], p["candidate_w"])), lin)
        q["gates_b"] = to(torch.cat((p["retention_b"], p["candidate_b"])))
        # feature logits of the key and of the query are linear in the states:
        # W_f (W_k x + b_k) + b_f = (W_f W_k) x + (W_f b_k + b_f), formed in float64
        f64 = lambda name: p[name].double()
        fk_w = f64("feature_w") @ f64("key_w")
        fk_b = f64("feature_w") @ f64("key_b") + f64("feature_b")
        fq_w = f64("feature_w") @ f64("query_w")
        fq_b = f64("feature_w") @ f64("query_b") + f64("feature_b")
        weights = [p["local_key_w"], p["local_value_w"], p["value_w"], fk_w, fq_w, p["decay_w"], p["write_w"]]
        biases = [p["local_key_b"], p["local_value_b"], p["value_b"], fk_b, fq_b, p["decay_b"], p["write_b"]]
        # rows padded (zero weights and biases) to a multiple of 4, so every row
        # of the projection starts 16-byte aligned for the kernels that read it,
        # and for a bf16 GEMM to a multiple of 256, whole tiles of the library's
        # 256-wide kernels (3108 -> 3328 columns at width 1024: a third less time)
        ws_w = torch.cat([w.double() for w in weights])
        ws_b = torch.cat([b.double() for b in biases])
        pad = -ws_w.shape[0] % (256 if lin == torch.bfloat16 else 4)
        q["ws_w"] = to(torch.cat((ws_w, ws_w.new_zeros((pad, ws_w.shape[1])))), lin)
        q["ws_b"] = to(torch.cat((ws_b, ws_b.new_zeros(pad))))
        q["fusion_w"], q["fusion_b"] = to(p["fusion_w"], lin), to(p["fusion_b"])
        if lin == torch.bfloat16:
            # the biases of GEMMs with bf16 results (nn.Linear under bf16 autocast)
            q["gates_b16"], q["ws_b16"], q["fusion_b16"] = (q[k].to(lin) for k in ("gates_b", "ws_b", "fusion_b"))
            q["fusion_b16f"] = q["fusion_b16"].float()  # the bf16 bias as the split fusion layer adds it
        q["fusion_norm"], q["expert_norm"] = to(p["fusion_norm"]), to(p["expert_norm"])
        for name in ("gate", "up", "down"):
            q[name + "_w"], q[name + "_b"] = to(p[name + "_w"], lin), to(p[name + "_b"], lin)
        if "router_w" in p:
            q["router_w"] = to(p["router_w"])
        if "refine_gate_w" in p:
            # the refine gate's [4 width] weight in the projections' dtype, its bias fp32
            q["refine_gate_w"] = to(p["refine_gate_w"].reshape(-1), lin)
            q["refine_gate_b"] = to(p["refine_gate_b"].reshape(1))
        q["head_w"], q["head_b"] = to(p["head_w"], lin), to(p["head_b"])
        q["content_w"] = to(p["head_w"][:PAD_TOKEN_ID])
        q["content_b"] = to(p["head_b"][:PAD_TOKEN_ID])
        if lin == torch.bfloat16:
            q["content_w16"] = q["content_w"].to(lin)
        prepared.append(q)
    return prepared


def add_decode_fragments(prepared: list[dict[str, Tensor]]) -> None:
    """Adds to each layer of a bf16 ``prepare_stack`` result the expert
    weights in fragment order (``gate_wf``, ``up_wf``, ``down_wf``; see
    ``moe.weights_to_fragments``), which the decode step's expert GEMMs then
    stream with contiguous loads. A second copy of the expert weights (the
    prefill keeps the row-major ones); results are unchanged bit for bit.
    Layers that already hold them, or whose experts are not bf16 MFMA shapes,
    are left as they are."""

    for q in prepared:
        w = q["gate_w"]
        if "gate_wf" in q or w.dtype != torch.bfloat16 or w.shape[1] % 64 or w.shape[2] % 64:
            continue
        for name in ("gate", "up", "down"):
            q[name + "_wf"] = moe.weights_to_fragments(q[name + "_w"])


def initial_states(settings: HermSettings, batch: int, device: torch.device) -> list[dict[str, Tensor]]:
    """KoemiState.create_static (state.py:43-76) per layer: zeros, rings at
    capacity with every slot invalid, last token PAD; with the herm ablation
    also the zero refine basis and normalizer."""

    d, m = settings.width, settings.memory_features
    w, s = settings.local_memory_size, settings.salience_memory_size
    states = []
    for _ in range(settings.layers):
        z = lambda *shape: torch.zeros(shape, device=device)
        refine = {"refine_basis": z(batch, d, m), "refine_normalizer": z(batch, m)} if settings.refine else {}
        states.append({
            **refine,
            "working": z(batch, d),
            "basis": z(batch, d, m),
            "normalizer": z(batch, m),
            "local_keys": z(batch, w, d),
            "local_values": z(batch, w, d),
            "local_valid": torch.zeros((batch, w), dtype=torch.bool, device=device),
            "salient_keys": z(batch, s, d),
            "salient_values": z(batch, s, d),
            "salient_valid": torch.zeros((batch, s), dtype=torch.bool, device=device),
            "last_token": torch.full((batch,), PAD_TOKEN_ID, dtype=torch.int64, device=device),
        })
    return states


def _rms(x: Tensor, weight: Tensor, residual: Tensor | None = None, mask: Tensor | None = None, *,
         fp32: bool = True, low: torch.dtype | None = None) -> Tensor | tuple[Tensor | None, Tensor | None]:
    """RootMeanSquareNorm.forward (layers.py:14-16) of ``x (+ residual)`` on
    ``koemi_herm_rmsnorm``; with ``mask``, rows whose mask is false keep ``x``
    (the expert mixture's valid-row select, experts.py:134-136). With ``low``
    (bf16) the kernel also writes that copy for a following GEMM and the call
    returns ``(fp32 or None, copy)``; ``fp32=False`` skips the fp32 output."""

    x = x.contiguous()
    width = x.shape[-1]
    out = torch.empty(x.shape, device=x.device, dtype=torch.float32) if fp32 or low is None else None
    out16 = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16) if low == torch.bfloat16 else None
    residual = residual.contiguous() if residual is not None else None
    mask = mask.contiguous() if mask is not None else None
    _native.call(
        "koemi_herm_rmsnorm", _native.ptr(x), _native.dtype_code(x.dtype),
        _native.ptr(residual) if residual is not None else None,
        _native.dtype_code(residual.dtype) if residual is not None else 0, _native.ptr(weight),
        _native.ptr(mask) if mask is not None else None, _native.ptr(out), _native.ptr(out16), x.numel() // width,
        width, _EPS, _native.stream_of(x.device),
    )
    if low is None:
        return out
    if out16 is None:  # no kernel-side copy for this dtype
        return out, out.to(low)
    return out, out16


def _linear(x: Tensor, weight: Tensor, bias: Tensor | None) -> Tensor:
    """x W^T (+ b) with fp32 results: for half-precision weights one library
    GEMM with fp32 accumulation and results, then the fp32 bias added in place
    (the library's fp32-output GEMM with a bias epilogue first copies the
    broadcast bias into the output and reads it back); ``x`` may already be in
    the weights' dtype (a copy its producer wrote). ``bias`` None: none (the
    gate biases are added inside the scan)."""

    if weight.dtype == torch.float32:
        return functional.linear(x, weight, bias)
    if _few_rows(x, weight):
        return linear.linear_rows([x], weight, bias)
    flat = x.reshape(-1, x.shape[-1]).to(weight.dtype)
    out = torch.mm(flat, weight.t(), out_dtype=torch.float32)
    if bias is not None:
        out += bias
    return out.view(*x.shape[:-1], weight.shape[0])


_GATE_STATUS: dict[int, Tensor] = {}


def gate_status(device: torch.device | str) -> Tensor:
    """The device's status word for the fused gate kernel inside captured
    graphs: ``recurrent.gated_projection_scan`` sets it to 1 when a tile's
    bounded wait for an earlier tile runs out (that tile's states are then
    NaN), and nothing clears it. Allocated on first use, which must come before
    any capture: every graph class of this module calls this in its
    constructor. Eager calls need no word (the front checks its own after the
    launch)."""

    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    word = _GATE_STATUS.get(index)
    if word is None:
        word = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda", index))
        _GATE_STATUS[index] = word
    return word


_BRANCH_STREAMS: dict[int, torch.cuda.Stream] = {}


def branch_stream(device: torch.device | str) -> torch.cuda.Stream:
    """The device's second stream (default priority) for the independent
    branches of a captured ``block_sequence``: the local and salient rings and
    reads run on it beside the associative memory on the capture stream, as
    parallel branches of the graph that join before the fusion layer.
    Created on first use, which must come before any capture (the graph
    classes call it in their constructors); a capture on a device without it
    runs the branches in turn."""

    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    stream = _BRANCH_STREAMS.get(index)
    if stream is None:
        stream = torch.cuda.Stream(device=torch.device("cuda", index))
        _BRANCH_STREAMS[index] = stream
    return stream


def check_gate_status(device: torch.device | str) -> None:
    """Raise ``recurrent.GatedScanTimeoutError`` if a captured fused gate
    kernel on ``device`` has reported a timed-out wait (a host sync)."""

    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    word = _GATE_STATUS.get(index)
    if word is not None:
        recurrent.check_gated_scan_status(word)


def _fused_gates(p: dict[str, Tensor], u: Tensor) -> bool:
    """Whether the gate projection and the scan run as the one fused kernel."""

    return p["gates_w"].dtype == torch.bfloat16 and recurrent.gated_projection_fits(u, p["gates_w"])


def _gated_scan(p: dict[str, Tensor], u: Tensor, valid: Tensor, working: Tensor, width: int, with_bf16: bool,
                out_bf16: Tensor | None, final_out: Tensor | None = None, states_out: Tensor | None = None):
    """The gate projection and the fused gates + scan: for a bf16 stack
    outside decode steps the projection's results are bf16 with the biases in
    the GEMM epilogue (nn.Linear under bf16 autocast) — in one kernel with the
    gates and the scan where the shape allows (whole 256-position tiles of a
    sequence), else a library GEMM then the scan kernel; otherwise fp32
    results without bias and the biases added inside the scan kernel.
    ``final_out``: where the fused kernel writes the last position's states
    (the next carried state), when that kernel runs; the caller checks
    ``_fused_gates(p, u)``. ``states_out``: the buffer for the states on the
    other paths (a decode graph's static state)."""

    w = p["gates_w"]
    if _fused_gates(p, u):
        status = None  # eager: the front checks its own status word after the launch
        if torch.cuda.is_current_stream_capturing():
            index = u.device.index if u.device.index is not None else torch.cuda.current_device()
            status = _GATE_STATUS.get(index)
            if status is None:
                raise RuntimeError("the fused gate kernel under graph capture needs herm.gate_status(device) "
                                   "allocated before the capture")
        return recurrent.gated_projection_scan(u, w, p["gates_b16"], valid, working, with_bf16=with_bf16,
                                               out_bf16=out_bf16, final_out=final_out, status=status)
    if u.shape[1] == 1 and w.dtype == torch.bfloat16 and _few_rows(u, w) and w.shape == (2 * width, u.shape[-1]):
        # a decode step: the gates and the one-position scan in the projection's epilogue
        batch = u.shape[0]
        states = states_out if states_out is not None else torch.empty((batch, 1, width), device=u.device,
                                                                        dtype=torch.float32)
        states16 = None
        if with_bf16:
            states16 = out_bf16 if out_bf16 is not None else torch.empty((batch, 1, width), device=u.device,
                                                                         dtype=torch.bfloat16)
        x = u.contiguous()
        _native.call("koemi_linear_rows_gated", _native.ptr(x), _native.dtype_code(x.dtype), _native.ptr(w),
                     _native.ptr(p["gates_b"][:width]), _native.ptr(p["gates_b"][width:]), _native.ptr(valid),
                     _native.ptr(working.contiguous()), _native.ptr(states), _native.ptr(states16),
                     states16.stride(1) if states16 is not None else 0, batch, width, x.shape[-1],
                     _native.stream_of(u.device))
        return (states, states16) if with_bf16 else states
    if w.dtype == torch.bfloat16 and not _few_rows(u, w):
        return recurrent.gated_scan(_linear_low(u, w, p["gates_b16"]), valid, working, width=width,
                                    with_bf16=with_bf16, out_bf16=out_bf16, out=states_out)
    return recurrent.gated_scan(_linear(u, w, None), valid, working, width=width, with_bf16=with_bf16,
                                retention_bias=p["gates_b"][:width], candidate_bias=p["gates_b"][width:],
                                out_bf16=out_bf16, out=states_out)


def _fusion_input(settings: HermSettings, batch: int, length: int, device: torch.device) -> Tensor | None:
    """The fusion layer's bf16 input [working ; memory ; local ; salient]
    (network.py:401-405) of a bf16 window of more than one position, written
    column block by column block by the scan's bf16 copy, the associative
    read and the two memory reads (no separate concatenation); None for fp32
    stacks and decode steps (their pieces are concatenated)."""

    if settings.linear_dtype != torch.bfloat16 or length == 1:
        return None
    return torch.empty((batch, length, 4 * settings.width), device=device, dtype=torch.bfloat16)


def _block(fusion_in: Tensor | None, index: int, width: int) -> Tensor | None:
    """Column block ``index`` (width columns) of the fusion input, or None."""

    return None if fusion_in is None else fusion_in[..., index * width:(index + 1) * width]


def _linear_low(x: Tensor, weight: Tensor, bias_low: Tensor) -> Tensor:
    """x W^T + b with bf16 results, the bias in the library GEMM's epilogue:
    nn.Linear under bf16 autocast (the reference's default GPU precision).
    Used for the working-state projection and the fusion layer of windows
    (not decode steps), whose consumers read bf16."""

    flat = x.reshape(-1, x.shape[-1])
    return torch.addmm(bias_low, flat, weight.t()).view(*x.shape[:-1], weight.shape[0])


def _projection(x: Tensor, p: dict[str, Tensor], name: str) -> Tensor:
    """The ``name`` projection (``ws`` or ``fusion``) of x: bf16 results for a
    bf16 stack outside decode steps, fp32 otherwise."""

    w = p[name + "_w"]
    if w.dtype == torch.bfloat16 and not _few_rows(x, w):
        return _linear_low(x, w, p[name + "_b16"])
    return _linear(x, w, p[name + "_b"]).contiguous()


def _few_rows(x: Tensor, weight: Tensor) -> bool:
    """Decode-step projections: a few rows and K <= 1024 (one or two staged
    chunks; the 4096-wide fusion input stays on the library GEMM)."""

    return (weight.dtype == torch.bfloat16 and x.numel() // x.shape[-1] <= linear.MAX_ROWS
            and x.shape[-1] % 64 == 0 and x.shape[-1] <= 1024 and x.dtype in (torch.float32, torch.bfloat16))


def _token_context(ids: Tensor, valid: Tensor | None, carried: Tensor, last_out: Tensor | None = None
                   ) -> tuple[Tensor, Tensor] | tuple[Tensor, Tensor, Tensor, Tensor]:
    """The previous valid token of each position and the last valid token of
    each row (network.py:742-761) on ``koemi_herm_token_context``. With
    ``valid`` None the kernel also forms the validity ``ids != PAD`` and the
    surprise targets (ids, 0 where invalid) and the call returns
    ``(previous, last, valid, targets)``. ``last_out``: the buffer that
    receives the last tokens (a graph's static state)."""

    batch, length = ids.shape
    previous = torch.empty_like(ids)
    last = torch.empty_like(carried) if last_out is None else last_out
    formed = valid is None
    valid_out = torch.empty(ids.shape, device=ids.device, dtype=torch.bool) if formed else None
    targets = torch.empty_like(ids) if formed else None
    _native.call("koemi_herm_token_context", _native.ptr(ids), _native.ptr(valid), _native.ptr(carried),
                 _native.ptr(previous), _native.ptr(last), _native.ptr(valid_out), _native.ptr(targets), PAD_TOKEN_ID,
                 batch, length, _native.stream_of(ids.device))
    return (previous, last, valid_out, targets) if formed else (previous, last)


def associative_scan_read(projections: Tensor, surprise: Tensor, valid: Tensor, basis: Tensor, normalizer: Tensor,
                          *, width: int, features: int, out: Tensor | None = None,
                          next_out: tuple[Tensor, Tensor] | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """The associative memory of one window on ``koemi_assoc_scan_read``:
    projection tail, fast write terms with the write masking and
    scan_and_read (memory.py:82-144, 244-255; network.py:734-740).

    ``projections`` fp32 ``[B, L, C]``, C >= 3 D + 2 M + 2, the stacked
    working-state projection: local key, local value and value pre-activations
    (D columns each), the feature logits of the key and of the query (M each;
    W_f W_k and W_f W_q folded into the projection) and the decay and write
    logits; columns past those (row padding) are not read.
    ``surprise`` ``[B, L]`` fp32, ``valid`` ``[B, L]`` bool, ``basis``
    ``[B, D, M]``, ``normalizer`` ``[B, M]`` fp32. Returns (reads ``[B, L, D]``,
    next basis, next normalizer); with ``out`` (an fp32 or bf16 ``[B, L, D]``
    view with evenly spaced rows, L > 1) the reads are written there, with
    ``next_out`` (contiguous buffers) the next basis and normalizer.
    """

    batch, length, stride = projections.shape
    d, m = width, features
    if (stride < 3 * d + 2 * m + 2 or projections.dtype not in (torch.float32, torch.bfloat16)
            or not projections.is_contiguous()):
        raise ValueError("projections must be contiguous fp32 or bf16 [batch, length, >= 3 * width + 2 * features + 2]")
    read = torch.empty((batch, length, d), device=projections.device, dtype=torch.float32) if out is None else out
    read_stride = memory._row_stride(read, (batch, length, d))
    next_basis, next_normalizer = next_out if next_out is not None else (torch.empty_like(basis),
                                                                         torch.empty_like(normalizer))
    need = _native.query("koemi_assoc_scan_read_workspace_bytes", batch, length, d, m)
    workspace = torch.empty((need,), device=projections.device, dtype=torch.uint8) if need else None
    args = [t.contiguous() for t in (surprise, valid, basis, normalizer)]
    _native.call(
        "koemi_assoc_scan_read",
        _native.ptr(projections), _native.dtype_code(projections.dtype), stride, 2 * d, 3 * d, 3 * d + m,
        3 * d + 2 * m, 3 * d + 2 * m + 1,
        *(_native.ptr(t) for t in args),
        _native.ptr(read), _native.dtype_code(read.dtype), read_stride, _native.ptr(next_basis),
        _native.ptr(next_normalizer),
        batch, length, d, m, _native.ptr(workspace), need, _native.stream_of(projections.device),
    )
    return read, next_basis, next_normalizer


def associative_refine_scan_read(projections: Tensor, surprise: Tensor, valid: Tensor, novelty: Tensor,
                                 fast: Tensor, basis: Tensor, normalizer: Tensor, *, width: int, features: int,
                                 rate: float, window: int | None = None,
                                 next_out: tuple[Tensor, Tensor] | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """The refine memory of the herm ablation (network.py:359-384) on
    ``koemi_assoc_refine_scan_read`` (or, with ``window``, over every window of
    a sequence on ``koemi_assoc_refine_scan_read_windows``): the write terms of
    memory.py:257-268 from the same ``projections`` as
    ``associative_scan_read``, ``surprise``, the local read's ``novelty``
    [B, L] fp32 and the fast reads ``fast`` [B, L, D] (fp32 or bf16, rows
    evenly spaced; the reconstruction error is clamp(tanh(v) - fast, -2, 2)),
    read from and written into the refine state ``basis`` [B, D, M] /
    ``normalizer`` [B, M]. Returns (refine reads [B, L, D] fp32, next basis,
    next normalizer); ``next_out`` as for ``associative_scan_read``."""

    batch, length, stride = projections.shape
    d, m = width, features
    if (stride < 3 * d + 2 * m + 2 or projections.dtype not in (torch.float32, torch.bfloat16)
            or not projections.is_contiguous()):
        raise ValueError("projections must be contiguous fp32 or bf16 [batch, length, >= 3 * width + 2 * features + 2]")
    if length == 1 and (fast.dtype != torch.float32 or not fast.is_contiguous()):
        fast = fast.float().contiguous()
    fast_stride = memory._row_stride(fast, (batch, length, d))
    read = torch.empty((batch, length, d), device=projections.device, dtype=torch.float32)
    next_basis, next_normalizer = next_out if next_out is not None else (torch.empty_like(basis),
                                                                         torch.empty_like(normalizer))
    args = [t.contiguous() for t in (surprise, valid, novelty)]
    state = [basis.contiguous(), normalizer.contiguous()]
    head = (_native.ptr(projections), _native.dtype_code(projections.dtype), stride, 2 * d, 3 * d, 3 * d + m,
            3 * d + 2 * m, 3 * d + 2 * m + 1, *(_native.ptr(t) for t in args), float(rate), _native.ptr(fast),
            _native.dtype_code(fast.dtype), fast_stride, *(_native.ptr(t) for t in state), _native.ptr(read),
            _native.dtype_code(read.dtype), d, _native.ptr(next_basis), _native.ptr(next_normalizer))
    if window is None:
        need = _native.query("koemi_assoc_refine_scan_read_workspace_bytes", batch, length, d, m)
        workspace = torch.empty((need,), device=projections.device, dtype=torch.uint8) if need else None
        _native.call("koemi_assoc_refine_scan_read", *head, batch, length, d, m, _native.ptr(workspace), need,
                     _native.stream_of(projections.device))
    else:
        if length % window:
            raise ValueError("the sequence length must be a multiple of the window")
        windows = length // window
        need = _native.query("koemi_assoc_refine_scan_read_windows_workspace_bytes", batch, windows, window, d, m)
        workspace = torch.empty((need,), device=projections.device, dtype=torch.uint8)
        _native.call("koemi_assoc_refine_scan_read_windows", *head, batch, windows, window, d, m,
                     _native.ptr(workspace), need, _native.stream_of(projections.device))
    return read, next_basis, next_normalizer


def _refine_gate(p: dict[str, Tensor], ws: Tensor, fast: Tensor, refine: Tensor, local: Tensor,
                 out: Tensor | None, low) -> Tensor:
    """KoemiModel.refine_memory (network.py:714-721) on
    ``koemi_herm_refine_gate``: the memory value fast + sigmoid(W_g [ws; fast;
    refine; local] + b_g) refine, [B, L, D], into ``out`` (the fusion input's
    memory block) or a new fp32 tensor. ``low`` (bf16 stacks) rounds the
    gate's inputs and pre-activation to bf16 (nn.Linear under autocast)."""

    batch, length, d = ws.shape
    value = torch.empty((batch, length, d), device=ws.device, dtype=torch.float32) if out is None else out
    pieces = (ws, fast, refine, local)
    if any(t.dtype != torch.float32 for t in pieces[:3]):
        raise ValueError("the refine gate takes fp32 working states, fast and refine reads")
    strides = [memory._row_stride(t, (batch, length, d)) for t in pieces] + [memory._row_stride(value,
                                                                                                (batch, length, d))]
    w = p["refine_gate_w"]
    _native.call("koemi_herm_refine_gate", _native.ptr(ws), strides[0], _native.ptr(fast), strides[1],
                 _native.ptr(refine), strides[2], _native.ptr(local), _native.dtype_code(local.dtype), strides[3],
                 _native.ptr(w), _native.dtype_code(w.dtype), _native.ptr(p["refine_gate_b"]), int(low is not None),
                 _native.ptr(value), _native.dtype_code(value.dtype), strides[4], batch * length, d,
                 _native.stream_of(ws.device))
    return value


class NextInput(NamedTuple):
    """A block's output handed to the next block of a stack already through
    that block's input RMSNorm: ``normalized`` [B, L, D] bf16, written by the
    fused expert tail (``koemi_herm_combine_norm``) in place of the fp32 final
    context, which nothing else reads between two blocks."""

    normalized: Tensor


def _input_norm(p: dict[str, Tensor], ids: Tensor, context, low) -> Tensor:
    """The block's input RMSNorm of its context (the embedding of the ids for
    the first block; a ``NextInput`` is already normalized): fp32, or the bf16
    copy for a bf16 stack."""

    if isinstance(context, NextInput):
        return context.normalized
    source = functional.embedding(ids, p["embedding"]) if context is None else context
    return _rms(source, p["input_norm"]) if low is None else _rms(source, p["input_norm"], fp32=False, low=low)[1]


_FUSION_SPLITS = 8  # K = 4 x 1024 fp32 inputs in 512-wide chunks: 8 x 32 workgroups


def _fusion_split_fits(p: dict[str, Tensor], pieces: tuple[Tensor, ...], d: int) -> bool:
    """Whether the fusion layer of a bf16 stack runs as a split-K projection
    of its four fp32 pieces (a decode step's few rows)."""

    w = p["fusion_w"]
    rows = pieces[0].numel() // d
    return (w.dtype == torch.bfloat16 and "fusion_b16" in p and len(pieces) == 4 and d % 1024 == 0
            and w.shape == (d, 4 * d) and rows <= linear.MAX_ROWS
            and all(t.dtype == torch.float32 and t.is_contiguous() and t.numel() == rows * d for t in pieces))


def _fusion_split(p: dict[str, Tensor], pieces: tuple[Tensor, ...], d: int) -> tuple[Tensor, Tensor]:
    """The fusion layer and its normalizer (network.py:401-405, 723-732) for a
    few rows: the four fp32 pieces [working ; memory ; local ; salient] are
    the K blocks of a split-K projection (no concatenation, the rows rounded
    to bf16 as staged), whose partial sums the norm kernel adds with the bf16
    bias and rounds to the bf16 result before normalizing. Returns (fp32,
    bf16) normalized rows in the pieces' shape."""

    shape = pieces[0].shape
    rows = pieces[0].numel() // d
    device = pieces[0].device
    partials = torch.empty((_FUSION_SPLITS, rows, d), device=device, dtype=torch.float32)
    stream = _native.stream_of(device)
    _native.call("koemi_linear_rows_split", *(_native.ptr(t) for t in pieces), 4, d,
                 _native.dtype_code(torch.float32), _native.ptr(p["fusion_w"]), None, _native.ptr(partials), rows, d,
                 _FUSION_SPLITS, stream)
    bias = p.get("fusion_b16f")
    if bias is None:
        bias = p["fusion_b16"].float()
    out = torch.empty(shape, device=device, dtype=torch.float32)
    out16 = torch.empty(shape, device=device, dtype=torch.bfloat16)
    _native.call("koemi_herm_rmsnorm_parts", _native.ptr(partials), _FUSION_SPLITS, _native.ptr(bias), 1,
                 _native.ptr(p["fusion_norm"]), _native.ptr(out), _native.ptr(out16), rows, d, _EPS, stream)
    return out, out16


def _fuse_mix_predict(p: dict[str, Tensor], settings: HermSettings, ids: Tensor, previous: Tensor, valid: Tensor,
                      pieces: tuple[Tensor, Tensor, Tensor, Tensor] | Tensor, with_logits: bool,
                      next_norm: Tensor | None = None, routing: dict | None = None
                      ) -> tuple[Tensor | NextInput, Tensor | None]:
    """The block's position-wise tail: fusion of [working ; memory ; local ;
    salient] with its normalizer (network.py:723-732), the expert mixture with
    its output normalizer (experts.py:109-150 or router.py:43-97) and the token
    head (network.py:700-701). Every position independent of the others, so
    the rows may span any number of windows. ``pieces`` are the four fp32
    inputs, or the bf16 fusion input their producers already wrote
    ([B, L, 4 D], see ``_fusion_input``). Returns (final context [B, L, D]
    fp32, logits or None). With ``next_norm`` (the next block's input norm
    weight) and a bf16 stack, the combine, this block's expert normalizer and
    the next block's input norm run as one kernel and the context returned is
    that ``NextInput`` (no fp32 context unless logits are asked for too).
    ``routing``: a dict shared by the layers of one stack pass; the hash
    route depends only on the ids and the validity (experts.py:283-289), so
    the first layer's permutation is kept there and reused by the others.
    With learned routing every call appends its ``moe.RouterStatistics``
    (router.py:50-58) to ``routing["statistics"]`` (the reference's
    KoemiOutput.router_statistics of a window; merge them with
    ``moe.merge_router_statistics``)."""

    batch, length = ids.shape
    d = settings.width
    k = settings.top_k
    lin = settings.linear_dtype
    low = lin if lin == torch.bfloat16 else None
    # bf16 MFMA shapes: the first expert GEMM reads the context rows by the
    # permutation's indices (no sorted copy of the context); hash routing is
    # then done inside the permutation (no assignments tensor)
    indexed = low is not None and d % 64 == 0 and p["gate_w"].shape[1] % 64 == 0
    hashed = indexed and settings.expert_routing != "learned"
    tail = low is not None and k <= 8 and d % 4 == 0 and d <= 2048  # the combined expert tail below
    fusion_rows = None  # bf16 fusion output whose fp32 normalized copy the expert tail forms itself
    if not isinstance(pieces, Tensor) and _fusion_split_fits(p, pieces, d):
        fused, fused_low = _fusion_split(p, pieces, d)
    else:
        if isinstance(pieces, Tensor):
            fusion_in = pieces
        elif low is None:
            fusion_in = torch.cat(pieces, dim=-1)
        else:
            fusion_in = torch.empty((batch, length, 4 * d), device=ids.device, dtype=low)
            _native.call("koemi_herm_concat_bf16", *(_native.ptr(t.contiguous()) for t in pieces), 4,
                         batch * length, d, _native.ptr(fusion_in), _native.stream_of(ids.device))
        projected = _projection(fusion_in, p, "fusion")
        if hashed and tail and projected.dtype == torch.bfloat16:
            # only the bf16 normalized rows are written here (the experts'
            # input); koemi_herm_combine_norm_fusion forms the fp32 ones
            fusion_rows = projected.reshape(-1, d)
            fused, fused_low = None, _rms(projected, p["fusion_norm"], fp32=False, low=low)[1]
        else:
            fused_pair = _rms(projected, p["fusion_norm"], low=low)
            fused, fused_low = fused_pair if low is not None else (fused_pair, None)

    flat = fused.reshape(-1, d) if fused is not None else None
    tokens = batch * length
    flat_valid = valid.reshape(-1)
    moe_in = fused_low.reshape(-1, d) if fused_low is not None else flat.to(lin)
    if settings.expert_routing == "learned":
        # LearnedExpertMixture (router.py:43-97): the bias-free gate on the fp32
        # context (rows of invalid tokens are routed to -1 whatever their
        # logits), softmax top-k, each pair weighted by its probability
        router_logits = functional.linear(flat, p["router_w"])
        assignments, weights, statistics = moe.route_topk_learned(router_logits, flat_valid, top_k=k,
                                                                  return_statistics=True)
        if routing is not None:  # the caller's RouterStatistics, one per learned block call
            routing.setdefault("statistics", []).append(statistics)
    elif not hashed:
        assignments = moe.route_topk_valid(ids, previous, valid, expert_count=settings.expert_count, top_k=k,
                                           validate=False)
        weights = None
    pair_positions = None
    if hashed:
        route = routing.get("hash") if routing is not None else None
        if route is None:
            route = moe.permute_hash_indices(ids, previous, flat_valid, expert_count=settings.expert_count, top_k=k)
            if routing is not None:
                routing["hash"] = route
        sorted_rows, sorted_experts, offsets, sorted_weights, pair_positions = route
    elif indexed:
        sorted_rows, sorted_experts, offsets, sorted_weights, pair_positions = moe.permute_indices(
            assignments.reshape(-1, k), flat_valid, expert_count=settings.expert_count, pair_weights=weights)
    else:
        permuted = moe.permute_topk(moe_in, assignments.reshape(-1, k), flat_valid,
                                    expert_count=settings.expert_count, pair_weights=weights, validate=False)
        sorted_context, sorted_rows, sorted_experts, offsets = permuted[:4]
        sorted_weights = permuted[4] if weights is not None else None
    if indexed and "gate_wf" in p and sorted_rows.shape[0] <= moe.FEW_PAIRS_PER_EXPERT * settings.expert_count:
        # a decode step's few rows per expert: the weights in fragment order
        # (add_decode_fragments), the same results as the indexed call below
        expert_out = moe.grouped_expert_mlp_fragments(moe_in, sorted_rows, offsets, p["gate_wf"], p["gate_b"],
                                                      p["up_wf"], p["up_b"], p["down_wf"], p["down_b"])
    elif indexed:
        expert_out = moe.grouped_expert_mlp_indexed(moe_in, sorted_rows, offsets, p["gate_w"], p["gate_b"],
                                                    p["up_w"], p["up_b"], p["down_w"], p["down_b"])
    else:
        expert_out = moe.grouped_expert_mlp_inference(sorted_context, sorted_experts, offsets, p["gate_w"],
                                                      p["gate_b"], p["up_w"], p["up_b"], p["down_w"], p["down_b"],
                                                      validate=False)
    if tail:
        # the combine, the expert normalizer and (inside a stack) the next
        # block's input norm in one kernel
        device = ids.device
        final = (torch.empty((tokens, d), device=device, dtype=torch.float32)
                 if with_logits or next_norm is None else None)
        u_next = torch.empty((tokens, d), device=device, dtype=torch.bfloat16) if next_norm is not None else None
        if fusion_rows is not None and pair_positions is not None:
            _native.call("koemi_herm_combine_norm_fusion", _native.ptr(expert_out), _native.ptr(pair_positions),
                         _native.ptr(offsets), _native.ptr(sorted_weights), _native.ptr(fusion_rows),
                         _native.ptr(p["fusion_norm"]), _native.ptr(flat_valid), _native.ptr(p["expert_norm"]),
                         _native.ptr(next_norm), _native.ptr(final), _native.ptr(u_next), int(expert_out.shape[0]),
                         d, tokens, k, settings.expert_count, _EPS, _native.stream_of(device))
        else:
            if flat is None:  # the fp32 normalized fusion rows after all
                flat = _rms(fusion_rows, p["fusion_norm"])
            need = _native.query("koemi_moe_combine_workspace_bytes", tokens, k) if pair_positions is None else 0
            workspace = torch.empty((need,), device=device, dtype=torch.uint8) if need else None
            _native.call("koemi_herm_combine_norm", _native.ptr(expert_out), _native.ptr(sorted_rows),
                         _native.ptr(pair_positions), _native.ptr(offsets), _native.ptr(sorted_weights),
                         _native.ptr(flat.contiguous()),
                         _native.ptr(flat_valid), _native.ptr(p["expert_norm"]), _native.ptr(next_norm),
                         _native.ptr(final), _native.ptr(u_next), int(expert_out.shape[0]), d, tokens, k,
                         settings.expert_count, _EPS, _native.ptr(workspace), need, _native.stream_of(device))
        logits = _linear(final.view(batch, length, d), p["head_w"], p["head_b"]) if with_logits else None
        if next_norm is None:
            return final.view(batch, length, d), logits
        return NextInput(u_next.view(batch, length, d)), logits
    update = moe.combine_topk(expert_out, sorted_rows, offsets, token_count=flat.shape[0], top_k=k,
                              pair_weights=sorted_weights, validate=False)
    final = _rms(flat, p["expert_norm"], residual=update, mask=flat_valid).view(batch, length, d)
    logits = _linear(final, p["head_w"], p["head_b"]) if with_logits else None
    return final, logits


def block_window(p: dict[str, Tensor], settings: HermSettings, ids: Tensor, state: dict[str, Tensor],
                 context: Tensor | NextInput | None = None, *, with_logits: bool = True,
                 token_context: tuple[Tensor, Tensor, Tensor, Tensor] | None = None,
                 next_norm: Tensor | None = None, out_state: dict[str, Tensor] | None = None,
                 routing: dict | None = None, surprise_in: tuple[Tensor, Tensor] | None = None
                 ) -> tuple[Tensor | None, Tensor | NextInput, dict[str, Tensor], Tensor]:
    """One forward_window of one block (network.py:296-441). ``ids`` ``[B, L]``
    int64 on the device; ``context`` the previous layer's final context (None
    for the embedding layer; a ``NextInput`` is taken as this block's
    normalized input). Returns (logits, final_context, next_state, surprise);
    logits is None when ``with_logits`` is False (the stack's inner layers,
    whose head output nothing reads). ``token_context``:
    ``_token_context``'s four outputs when the caller formed them (a decode
    step's stack, once for all layers). ``next_norm``: the next block's input
    norm weight, for a stack; the context returned is then a ``NextInput``
    (see ``_fuse_mix_predict``). ``out_state`` (a decode step, one position):
    a state dict whose buffers receive the next state (a decode graph's other
    static state; ``last_token`` is the caller's, from the token context).
    ``routing``: shared by the layers of a stack pass (see
    ``_fuse_mix_predict``). ``surprise_in``: this layer's (surprise,
    admission) [B, 1] when the caller formed them (a decode step's stack, all
    layers at once: they depend on the carried states alone)."""

    ids = ids.contiguous()
    batch, length = ids.shape
    d = settings.width
    # validity, surprise targets and the routing context of every position in one kernel
    if token_context is None:
        token_context = _token_context(ids, None, state["last_token"])
    previous, last_token, valid, targets = token_context
    lin = settings.linear_dtype
    low = lin if lin == torch.bfloat16 else None  # kernels write bf16 copies of the GEMM inputs
    u = _input_norm(p, ids, context, low)
    fusion_in = _fusion_input(settings, batch, length, ids.device)
    if out_state is not None and (length != 1 or _fused_gates(p, u)):
        raise ValueError("out_state is for decode steps (one position)")
    states_out = out_state["working"].view(batch, 1, d) if out_state is not None else None
    scanned = _gated_scan(p, u, valid, state["working"], d, low is not None, _block(fusion_in, 0, d),
                          states_out=states_out)
    ws, ws_low = scanned if low is not None else (scanned, scanned)
    if surprise_in is not None and length == 1:
        surprise, admission = surprise_in
    else:
        surprise, admission = _surprise_after(p, settings, ws, ws_low, state["working"], targets, valid)

    projected = _projection(ws_low, p, "ws")
    # local keys and values: the first two column blocks, read in place (the
    # rings zero invalid entries on the way; the reads never see them)
    local_keys, local_values = projected[..., :d], projected[..., d:2 * d]
    ring_out = lambda name: (None if out_state is None else
                             tuple(out_state[name + part] for part in ("_keys", "_values", "_valid")))
    if state["local_keys"].shape[1] != settings.local_memory_size:
        raise ValueError("the local ring must hold exactly `local_memory_size` entries (static state)")
    step_rings = (length == 1 and state["salient_keys"].shape[1] == settings.salience_memory_size
                  and all(state[k].is_contiguous() for k in ("local_keys", "local_values", "local_valid",
                                                              "salient_keys", "salient_values", "salient_valid")))
    assoc_done = False
    if length == 1:
        # a decode step: only the carried slots are eligible, both reads in one
        # launch, with both rings after the step when they are static (and
        # then the associative memory's step as well)
        local_value = torch.empty((batch, 1, d), device=ids.device, dtype=torch.float32)
        salient_value = torch.empty_like(local_value)
        common = (_native.ptr(state["local_keys"]), _native.ptr(state["local_values"]),
                  _native.ptr(state["local_valid"]), state["local_keys"].shape[1], settings.local_memory_size,
                  _native.ptr(state["salient_keys"]), _native.ptr(state["salient_values"]),
                  _native.ptr(state["salient_valid"]), state["salient_keys"].shape[1], _native.ptr(ws),
                  _native.ptr(local_value), _native.ptr(salient_value))
        if step_rings:
            local_ring = ring_out("local") or tuple(torch.empty_like(state["local" + part])
                                                    for part in ("_keys", "_values", "_valid"))
            salient = ring_out("salient") or tuple(torch.empty_like(state["salient" + part])
                                                   for part in ("_keys", "_values", "_valid"))
            m = settings.memory_features
            if (projected.is_contiguous() and m <= 32 and projected.shape[-1] >= 3 * d + 2 * m + 2
                    and not settings.refine):
                # the associative memory's step joins the same launch
                fast = torch.empty((batch, 1, d), device=ids.device, dtype=torch.float32)
                basis, normalizer = ((out_state["basis"], out_state["normalizer"]) if out_state is not None
                                     else (torch.empty_like(state["basis"]), torch.empty_like(state["normalizer"])))
                _native.call("koemi_decode_memory_step", *common, _native.ptr(projected),
                             _native.dtype_code(projected.dtype), projected.shape[-1], 0, d, _native.ptr(valid),
                             _native.ptr(admission), *(_native.ptr(t) for t in local_ring + salient), 2 * d, 3 * d,
                             3 * d + m, 3 * d + 2 * m, 3 * d + 2 * m + 1, _native.ptr(surprise.contiguous()),
                             _native.ptr(state["basis"].contiguous()), _native.ptr(state["normalizer"].contiguous()),
                             _native.ptr(fast), _native.ptr(basis), _native.ptr(normalizer), m, batch, d,
                             _native.stream_of(ids.device))
                assoc_done = True
            else:
                _native.call("koemi_read_step_pair_rings", *common, _native.ptr(local_keys),
                             _native.ptr(local_values), _native.dtype_code(local_keys.dtype), local_keys.stride(1),
                             _native.ptr(valid), _native.ptr(admission), *(_native.ptr(t) for t in local_ring + salient),
                             batch, d, _native.stream_of(ids.device))
        else:
            _native.call("koemi_read_step_pair", *common, batch, d, _native.stream_of(ids.device))
    else:
        local_value = memory.read_local_window(state["local_keys"], state["local_values"], state["local_valid"],
                                               local_keys, local_values, valid, ws, window=settings.local_memory_size,
                                               out=_block(fusion_in, 2, d))

    if not assoc_done:
        # with the refine memory the fast reads stay fp32 for the reconstruction
        # error and the gate; the memory value goes to the fusion input instead
        fast, basis, normalizer = associative_scan_read(
            projected, surprise, valid, state["basis"], state["normalizer"], width=d,
            features=settings.memory_features, out=None if settings.refine else _block(fusion_in, 1, d),
            next_out=(out_state["basis"], out_state["normalizer"]) if out_state is not None else None)
    refine_next = {}
    if settings.refine:
        # network.py:359-384: the local read's novelty, the refine terms and
        # their scan-and-read over the refine state, the refine gate
        novelty = memory.local_novelty(state["local_keys"], state["local_valid"], local_keys, valid, ws,
                                       window=settings.local_memory_size)
        refine, refine_basis, refine_normalizer = associative_refine_scan_read(
            projected, surprise, valid, novelty, fast, state["refine_basis"], state["refine_normalizer"], width=d,
            features=settings.memory_features, rate=settings.refine_decay_rate,
            next_out=(out_state["refine_basis"], out_state["refine_normalizer"]) if out_state is not None else None)
        local_in = local_value if fusion_in is None or length == 1 else _block(fusion_in, 2, d)
        fast = _refine_gate(p, ws, fast, refine, local_in, _block(fusion_in, 1, d), low)
        refine_next = {"refine_basis": refine_basis, "refine_normalizer": refine_normalizer}

    if length != 1:
        salient_value = memory.read_salient_window(state["salient_keys"], state["salient_values"],
                                                   state["salient_valid"], local_keys, local_values, admission, ws,
                                                   out=_block(fusion_in, 3, d))
    pieces = fusion_in if fusion_in is not None else (ws, fast, local_value, salient_value)
    final, logits = _fuse_mix_predict(p, settings, ids, previous, valid, pieces, with_logits, next_norm, routing)

    if not step_rings:
        _, local_ring = window_rings(state["local_keys"], state["local_values"], state["local_valid"], local_keys,
                                     local_values, valid, window=length, capacity=settings.local_memory_size,
                                     tail=True, key_valid=valid, final_only=True, final_out=ring_out("local"))
        _, salient = window_rings(state["salient_keys"], state["salient_values"], state["salient_valid"],
                                  local_keys, local_values, admission, window=length,
                                  capacity=settings.salience_memory_size, tail=False, key_valid=valid,
                                  final_only=True, final_out=ring_out("salient"))
    next_state = {
        "working": ws[:, -1].contiguous(),
        "basis": basis,
        "normalizer": normalizer,
        "local_keys": local_ring[0],
        "local_values": local_ring[1],
        "local_valid": local_ring[2],
        "salient_keys": salient[0],
        "salient_values": salient[1],
        "salient_valid": salient[2],
        "last_token": last_token,
        **refine_next,
    }
    return logits, final, next_state, surprise


def window_rings(carried_keys: Tensor, carried_values: Tensor, carried_flags: Tensor, keys: Tensor, values: Tensor,
                 flags: Tensor, *, window: int, capacity: int, tail: bool, key_valid: Tensor | None = None,
                 final_only: bool = False, final_out: tuple[Tensor, Tensor, Tensor] | None = None
                 ) -> tuple[tuple[Tensor, Tensor, Tensor] | None, tuple[Tensor, Tensor, Tensor]]:
    """The ring carried into every window of a sequence and the ring after it
    (``koemi_window_rings``): ``((keys, values, flags), (final keys, final
    values, final flags))`` with ``[B * L / window, capacity, D]`` keys and
    values and ``[B * L / window, capacity]`` flags (row ``b * L / window +
    w`` is the ring carried into window ``w`` of batch row ``b``, the layout
    the batched window reads take), and ``[B, capacity, ...]`` finals.
    ``tail``: the local ring (the last ``capacity`` entries,
    LocalKeyValueMemory.tail, memory.py:385-403); otherwise the salient ring
    (salient_tail, memory.py:431-455).

    ``keys``/``values`` ``[B, L, D]`` may be views with evenly spaced rows
    (column blocks of the block's projection, fp32 or bf16, read in place
    into fp32 rings); ``key_valid`` ``[B, L]`` zeroes the entries of invalid
    positions on the way (network.py:337-340). ``final_only``: only the ring
    after the sequence (the first result is None); ``final_out``: buffers
    that receive it (a decode graph's static state)."""

    batch, length, width = keys.shape
    rows = batch * (length // window)
    ring_dtype = carried_keys.dtype
    strided = keys.dtype != ring_dtype or not keys.is_contiguous() or not values.is_contiguous()
    if strided or key_valid is not None:
        stride = keys.stride(1)
        if (keys.stride(2) != 1 or keys.stride(0) != length * stride or values.stride() != keys.stride()
                or values.dtype != keys.dtype):
            raise ValueError("window ring entries must be views with contiguous columns and evenly spaced rows")
    else:
        keys, values = keys.contiguous(), values.contiguous()
        stride = width
    if final_only:
        out_k = out_v = out_ok = None
    else:
        out_k = torch.empty((rows, capacity, width), device=keys.device, dtype=ring_dtype)
        out_v = torch.empty_like(out_k)
        out_ok = torch.empty((rows, capacity), device=keys.device, dtype=torch.bool)
    slots = min(carried_keys.shape[1] + length, capacity)
    if final_out is not None:
        fin_k, fin_v, fin_ok = final_out
        if fin_k.shape != (batch, slots, width) or fin_ok.shape != (batch, slots) or not all(
                t.is_contiguous() for t in final_out):
            raise ValueError("final_out must be contiguous [B, slots, D], [B, slots, D] and [B, slots] buffers")
    else:
        fin_k = torch.empty((batch, slots, width), device=keys.device, dtype=ring_dtype)
        fin_v = torch.empty_like(fin_k)
        fin_ok = torch.empty((batch, slots), device=keys.device, dtype=torch.bool)
    ck, cv, cf, fl = (t.contiguous() for t in (carried_keys, carried_values, carried_flags, flags))
    kv = None if key_valid is None else key_valid.contiguous()
    _native.call("koemi_window_rings", _native.ptr(ck), _native.ptr(cv), _native.ptr(cf), _native.ptr(keys),
                 _native.ptr(values), _native.dtype_code(keys.dtype), stride, _native.ptr(kv), _native.ptr(fl),
                 _native.ptr(out_k), _native.ptr(out_v), _native.ptr(out_ok), _native.ptr(fin_k), _native.ptr(fin_v),
                 _native.ptr(fin_ok), batch, carried_keys.shape[1], length, window, width, capacity, int(tail),
                 _native.dtype_code(ring_dtype), _native.stream_of(keys.device))
    return (None if final_only else (out_k, out_v, out_ok)), (fin_k, fin_v, fin_ok)


def associative_scan_read_windows(projections: Tensor, surprise: Tensor, valid: Tensor, basis: Tensor,
                                  normalizer: Tensor, *, width: int, features: int, window: int,
                                  out: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """``associative_scan_read`` over every window of a sequence at once
    (``koemi_assoc_scan_read_windows``): the same inputs with length = a
    multiple of ``window``; each window reads from the state the previous
    windows left (equal to a window-by-window run's), and the state after the
    last window is returned with the reads."""

    batch, length, stride = projections.shape
    d, m = width, features
    if (stride < 3 * d + 2 * m + 2 or projections.dtype not in (torch.float32, torch.bfloat16)
            or not projections.is_contiguous()):
        raise ValueError("projections must be contiguous fp32 or bf16 [batch, length, >= 3 * width + 2 * features + 2]")
    if length % window:
        raise ValueError("the sequence length must be a multiple of the window")
    windows = length // window
    read = torch.empty((batch, length, d), device=projections.device, dtype=torch.float32) if out is None else out
    read_stride = memory._row_stride(read, (batch, length, d))
    next_basis = torch.empty_like(basis)
    next_normalizer = torch.empty_like(normalizer)
    workspace = torch.empty((_native.query("koemi_assoc_scan_read_windows_workspace_bytes", batch, windows, window, d,
                                           m),), device=projections.device, dtype=torch.uint8)
    args = [t.contiguous() for t in (surprise, valid, basis, normalizer)]
    _native.call(
        "koemi_assoc_scan_read_windows",
        _native.ptr(projections), _native.dtype_code(projections.dtype), stride, 2 * d, 3 * d, 3 * d + m,
        3 * d + 2 * m, 3 * d + 2 * m + 1,
        *(_native.ptr(t) for t in args),
        _native.ptr(read), _native.dtype_code(read.dtype), read_stride, _native.ptr(next_basis),
        _native.ptr(next_normalizer),
        batch, windows, window, d, m, _native.ptr(workspace), workspace.numel(), _native.stream_of(projections.device),
    )
    return read, next_basis, next_normalizer


def _surprise_carried(p: dict[str, Tensor], settings: HermSettings, carried: Tensor, targets: Tensor,
                      valid: Tensor) -> tuple[Tensor, Tensor]:
    """Surprise and admission of a one-position window ([B, 1]), which depend
    on the carried working state alone: its content logits (``linear_rows``
    for bf16 heads, a decode step's few rows) and the shifted surprise kernel
    at length 1."""

    batch = carried.shape[0]
    w16 = p.get("content_w16")
    if w16 is not None:
        first = linear.linear_rows([carried], w16, None)
    else:
        first = torch.mm(carried, p["content_w"].t())
    surprise = torch.empty((batch, 1), device=carried.device, dtype=torch.float32)
    admission = torch.empty((batch, 1), device=carried.device, dtype=torch.bool)
    vocab = first.shape[1]
    _native.call("koemi_herm_surprise_shifted", _native.ptr(first), _native.ptr(first), _native.ptr(p["content_b"]),
                 _native.ptr(targets), _native.ptr(valid), _native.ptr(surprise), _native.ptr(admission),
                 float(settings.salience_threshold), batch, 1, vocab, think._log_vocab(vocab),
                 _native.stream_of(carried.device))
    return surprise, admission


def _surprise_layers(params: list[dict[str, Tensor]], settings: HermSettings, states: list[dict[str, Tensor]],
                     targets: Tensor, valid: Tensor) -> list[tuple[Tensor, Tensor]] | None:
    """A decode step's surprise and admission in every layer at once: each
    depends only on the layer's carried working state (``_surprise_carried``),
    so the content heads of all layers run as one batched projection
    (``koemi_linear_rows_batched``) and the scoring as one kernel
    (``koemi_herm_surprise_layers``). None when the stack does not fit them
    (fp32 heads, another vocabulary, more than 32 layers)."""

    layers = len(params)
    w16 = [p.get("content_w16") for p in params]
    carried = [st["working"] for st in states]
    if layers > 32 or any(w is None for w in w16) or targets.shape[1] != 1:
        return None
    batch, d = carried[0].shape
    vocab = w16[0].shape[0]
    if (vocab != 256 or d % 64 or batch > linear.MAX_ROWS
            or any(w.shape != (vocab, d) or not w.is_contiguous() for w in w16)
            or any(c.shape != (batch, d) or c.dtype != torch.float32 or not c.is_contiguous() for c in carried)):
        return None
    biases = [p["content_b"] for p in params]
    if any(b.shape != (vocab,) or b.dtype != torch.float32 or not b.is_contiguous() for b in biases):
        return None
    device = carried[0].device
    logits = torch.empty((layers, batch, vocab), device=device, dtype=torch.float32)
    stream = _native.stream_of(device)
    _native.call("koemi_linear_rows_batched", _native.ptr_array(carried), _native.dtype_code(torch.float32),
                 _native.ptr_array(w16), None, _native.ptr(logits), layers, batch, d, vocab, stream)
    surprise = torch.empty((layers, batch, 1), device=device, dtype=torch.float32)
    admission = torch.empty((layers, batch, 1), device=device, dtype=torch.bool)
    _native.call("koemi_herm_surprise_layers", _native.ptr(logits), _native.ptr_array(biases),
                 _native.ptr(targets), _native.ptr(valid), _native.ptr(surprise), _native.ptr(admission),
                 float(settings.salience_threshold), layers, batch, vocab, think._log_vocab(vocab), stream)
    return [(surprise[layer], admission[layer]) for layer in range(layers)]


def _carried_logits(params: list[dict[str, Tensor]], states: list[dict[str, Tensor]]) -> list[Tensor] | None:
    """Every layer's content logits of its carried working state (the
    surprise of a sequence's first position, network.py:318-325), one batched
    projection for the stack (``koemi_linear_rows_batched``: the arithmetic of
    the per-layer ``linear_rows`` call, so the same bits) in place of a launch
    per layer. None when the stack does not fit it (fp32 heads, more than 32
    layers, rows the projection does not take)."""

    w16 = [p.get("content_w16") for p in params]
    carried = [st["working"] for st in states]
    if len(params) > 32 or any(w is None for w in w16):
        return None
    batch, d = carried[0].shape
    vocab = w16[0].shape[0]
    if (d % 64 or d > 1024 or batch > linear.MAX_ROWS
            or any(w.shape != (vocab, d) or not w.is_contiguous() for w in w16)
            or any(c.shape != (batch, d) or c.dtype != torch.float32 or not c.is_contiguous() for c in carried)):
        return None
    device = carried[0].device
    logits = torch.empty((len(params), batch, vocab), device=device, dtype=torch.float32)
    _native.call("koemi_linear_rows_batched", _native.ptr_array(carried), _native.dtype_code(torch.float32),
                 _native.ptr_array(w16), None, _native.ptr(logits), len(params), batch, d, vocab,
                 _native.stream_of(device))
    return [logits[layer] for layer in range(len(params))]


def _surprise_after(p: dict[str, Tensor], settings: HermSettings, ws: Tensor, ws_low: Tensor, carried: Tensor,
                    targets: Tensor, valid: Tensor, first: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """causal_surprise of every position from the state before it (the carried
    state, then the window's own; network.py:318-325, 677-698) and the
    fixed-threshold admission (network.py:349), without forming the shifted
    states: the content logits of the carried state and of every working
    state (fp32 results; bf16 operands for a bf16 stack, the content head under
    bf16 autocast), then one kernel (``koemi_herm_surprise_shifted``) scoring
    row t on the logits of row t - 1 (the carried state's for t = 0). Returns
    (surprise fp32 [B, L], admission bool [B, L]). ``first``: the carried
    state's content logits when the caller formed them (``_carried_logits``)."""

    batch, length, d = ws.shape
    if length == 1:
        return _surprise_carried(p, settings, carried, targets, valid)
    w16 = p.get("content_w16")
    if w16 is not None:
        weight_t = w16.t()
        # the carried state's few rows: one kernel (fp32 rows rounded to bf16 as staged)
        if first is None:
            first = linear.linear_rows([carried], w16, None) if _few_rows(carried, w16) else \
                torch.mm(carried.to(torch.bfloat16), weight_t, out_dtype=torch.float32)
        logits = torch.mm(ws_low.reshape(batch * length, d), weight_t, out_dtype=torch.float32) if length > 1 \
            else first
    else:
        weight_t = p["content_w"].t()
        first = torch.mm(carried, weight_t)
        logits = torch.mm(ws.reshape(batch * length, d), weight_t) if length > 1 else first
    surprise = torch.empty((batch, length), device=ws.device, dtype=torch.float32)
    admission = torch.empty((batch, length), device=ws.device, dtype=torch.bool)
    vocab = first.shape[1]
    _native.call("koemi_herm_surprise_shifted", _native.ptr(logits), _native.ptr(first), _native.ptr(p["content_b"]),
                 _native.ptr(targets), _native.ptr(valid), _native.ptr(surprise), _native.ptr(admission),
                 float(settings.salience_threshold), batch, length, vocab, think._log_vocab(vocab),
                 _native.stream_of(ws.device))
    return surprise, admission


def block_sequence(p: dict[str, Tensor], settings: HermSettings, ids: Tensor, state: dict[str, Tensor],
                   context: Tensor | NextInput | None = None, *, with_logits: bool = True,
                   token_context: tuple[Tensor, Tensor, Tensor, Tensor] | None = None,
                   next_norm: Tensor | None = None, routing: dict | None = None,
                   carried_logits: Tensor | None = None
                   ) -> tuple[Tensor | None, Tensor | NextInput, dict[str, Tensor], Tensor]:
    """One block over a whole sequence of windows at once: forward_parallel
    (network.py:176-197) of a single block, i.e. ``block_window`` applied to
    windows of ``scan_chunk`` tokens with the state carried, computed
    sequence-parallel. ``ids`` ``[B, L]``, L a multiple of ``scan_chunk``,
    static state rings (``initial_states``).

    No part of a window's carried state (working state, associative basis and
    normalizer, local and salient rings, last token) depends on the fusion,
    the experts or the head, so those run once over all positions, and so do
    the projections, the surprise head and the admission (position-wise).
    The recurrence runs as one scan over the whole sequence; the local and
    salient reads of all windows run as one batch of B x L / scan_chunk rows,
    each with the ring carried into its window (``window_rings``); the
    associative memory runs per window from the state the previous windows
    left (``associative_scan_read_windows``). The results equal the
    window-by-window ones up to floating-point rounding (the library GEMMs
    see more rows). ``token_context``: ``_token_context``'s four outputs when
    the caller formed them (a stack, once for all layers); ``context``,
    ``next_norm`` and ``routing`` as in ``block_window``; ``carried_logits``:
    the content logits of ``state["working"]`` when the caller formed them
    (``_carried_logits``, one launch for a stack). Returns (logits or None,
    final context, next state, surprise [B, L]).
    """

    ids = ids.contiguous()
    batch, length = ids.shape
    chunk, d = settings.scan_chunk, settings.width
    if length % chunk:
        raise ValueError("block_sequence needs a length that is a multiple of scan_chunk")
    windows = length // chunk
    rows = batch * windows
    if token_context is None:
        token_context = _token_context(ids, None, state["last_token"])
    previous, last_token, valid, targets = token_context
    lin = settings.linear_dtype
    low = lin if lin == torch.bfloat16 else None
    u = _input_norm(p, ids, context, low)
    fusion_in = _fusion_input(settings, batch, length, ids.device)
    working_next = torch.empty((batch, d), device=ids.device, dtype=torch.float32) if _fused_gates(p, u) else None
    scanned = _gated_scan(p, u, valid, state["working"], d, low is not None, _block(fusion_in, 0, d), working_next)
    ws, ws_low = scanned if low is not None else (scanned, scanned)
    surprise, admission = _surprise_after(p, settings, ws, ws_low, state["working"], targets, valid,
                                          carried_logits)

    projected = _projection(ws_low, p, "ws")
    # local keys and values read in place from the projection (see block_window)
    local_keys, local_values = projected[..., :d], projected[..., d:2 * d]
    cap_l, cap_s = settings.local_memory_size, settings.salience_memory_size
    per_window = lambda t: None if t is None else t.view(rows, chunk, *t.shape[2:])
    # Under capture the local and salient memories (rings and reads) form a
    # branch of the graph on the branch stream beside the associative memory
    # (the refine memory reads the local ring, so that ablation stays in turn).
    main = torch.cuda.current_stream(ids.device)
    side = None
    if not settings.refine and torch.cuda.is_current_stream_capturing():
        side = _BRANCH_STREAMS.get(ids.device.index if ids.device.index is not None else torch.cuda.current_device())
    if side is not None:
        side.wait_stream(main)

    def rings_and_reads():
        local_rings, local_final = window_rings(state["local_keys"], state["local_values"], state["local_valid"],
                                                local_keys, local_values, valid, window=chunk, capacity=cap_l,
                                                tail=True, key_valid=valid)
        local_value = memory.read_local_window(*local_rings, per_window(local_keys), per_window(local_values),
                                               per_window(valid), per_window(ws), window=cap_l,
                                               out=per_window(_block(fusion_in, 2, d)))
        salient_rings, salient_final = window_rings(state["salient_keys"], state["salient_values"],
                                                    state["salient_valid"], local_keys, local_values, admission,
                                                    window=chunk, capacity=cap_s, tail=False, key_valid=valid)
        salient_value = memory.read_salient_window(*salient_rings, per_window(local_keys), per_window(local_values),
                                                   per_window(admission), per_window(ws),
                                                   out=per_window(_block(fusion_in, 3, d)))
        return local_rings, local_final, local_value, salient_final, salient_value

    if side is not None:
        with torch.cuda.stream(side):
            local_rings, local_final, local_value, salient_final, salient_value = rings_and_reads()
    else:
        local_rings, local_final, local_value, salient_final, salient_value = rings_and_reads()
    fast, basis, normalizer = associative_scan_read_windows(projected, surprise, valid, state["basis"],
                                                            state["normalizer"], width=d,
                                                            features=settings.memory_features, window=chunk,
                                                            out=None if settings.refine else _block(fusion_in, 1, d))
    if side is not None:
        main.wait_stream(side)
    refine_next = {}
    if settings.refine:
        # the refine memory (network.py:359-384) of every window at once: each
        # window's novelty against the local ring it receives, the refine
        # terms' scan-and-read carried over the windows, the gate
        novelty = memory.local_novelty(local_rings[0], local_rings[2], per_window(local_keys), per_window(valid),
                                       per_window(ws), window=cap_l).view(batch, length)
        refine, refine_basis, refine_normalizer = associative_refine_scan_read(
            projected, surprise, valid, novelty, fast, state["refine_basis"], state["refine_normalizer"], width=d,
            features=settings.memory_features, rate=settings.refine_decay_rate, window=chunk)
        fast = _refine_gate(p, ws, fast, refine, local_value.view(batch, length, d), _block(fusion_in, 1, d), low)
        refine_next = {"refine_basis": refine_basis, "refine_normalizer": refine_normalizer}
    if fusion_in is not None:
        pieces = fusion_in
    else:
        pieces = (ws, fast, local_value.view(batch, length, d), salient_value.view(batch, length, d))
    final, logits = _fuse_mix_predict(p, settings, ids, previous, valid, pieces, with_logits, next_norm, routing)
    next_state = {
        "working": working_next if working_next is not None else ws[:, -1].contiguous(),
        "basis": basis,
        "normalizer": normalizer,
        "local_keys": local_final[0],
        "local_values": local_final[1],
        "local_valid": local_final[2],
        "salient_keys": salient_final[0],
        "salient_values": salient_final[1],
        "salient_valid": salient_final[2],
        "last_token": last_token,
        **refine_next,
    }
    return logits, final, next_state, surprise


def stack_sequence(params: list[dict[str, Tensor]], settings: HermSettings, ids: Tensor,
                   states: list[dict[str, Tensor]], surprise_out: list[Tensor] | None = None
                   ) -> tuple[Tensor, list[dict[str, Tensor]]]:
    """``prefill`` computed layer by layer with ``block_sequence``: each layer
    over the whole sequence before the next. The token context (validity,
    previous tokens, surprise targets) is formed once for all layers: every
    layer sees the same ids and carries the same last token. Returns the last
    layer's logits of every position and the next states; ``surprise_out``
    (a list) receives every layer's surprise [B, L] (the admission mask is
    ``valid & (surprise > threshold)``, network.py:349)."""

    ids = ids.contiguous()
    token_context = _token_context(ids, None, states[0]["last_token"])
    context = None
    next_states = []
    logits = None
    routing: dict = {}  # the hash route, formed by the first layer for all of them
    # every layer's carried-state content logits in one launch (they depend
    # only on the starting states)
    carried = _carried_logits(params, states) if ids.shape[1] > 1 else None
    for layer, (p, state) in enumerate(zip(params, states)):
        last = layer == len(params) - 1
        logits, context, next_state, surprise = block_sequence(
            p, settings, ids, state, context, with_logits=last, token_context=token_context,
            next_norm=None if last else params[layer + 1]["input_norm"], routing=routing,
            carried_logits=None if carried is None else carried[layer])
        next_states.append(next_state)
        if surprise_out is not None:
            surprise_out.append(surprise)
    return logits, next_states


class SequencePrefill:
    """``stack_sequence`` at a fixed (batch, length) replayed from one captured
    HIP graph. The graph reads the ids and the starting states from static
    buffers it never writes (``self.start``: the states given at
    construction) and writes the logits and the states after the sequence
    (``self.states``) into buffers of its own, so a replay needs no copies:
    ``run(ids=None, states=None)`` copies in only what is given (ids other
    than the static ids buffer; starting states, which then stay the start
    of later runs), replays, and returns the logits buffer; ``self.surprise``
    holds every layer's surprise of the last replay. Two eager passes
    on throwaway copies warm the libraries up before the capture. The fused
    gate kernel reports a timed-out wait into ``self.status`` (NaN states,
    never silently wrong ones): ``check()`` raises if that happened in any
    replay so far."""

    def __init__(self, params: list[dict[str, Tensor]], settings: HermSettings, states: list[dict[str, Tensor]],
                 ids: Tensor) -> None:
        self.params, self.settings = params, settings
        self.ids = ids.clone().contiguous()
        self.status = gate_status(self.ids.device)
        branch_stream(self.ids.device)
        self.start = [{k: v.clone() for k, v in st.items()} for st in states]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            warm = [{k: v.clone() for k, v in st.items()} for st in states]
            for _ in range(2):
                stack_sequence(params, settings, self.ids, warm)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        self.surprise: list[Tensor] = []
        with torch.cuda.graph(self.graph):
            self.logits, self.states = stack_sequence(params, settings, self.ids, self.start, self.surprise)

    def run(self, ids: Tensor | None = None, states: list[dict[str, Tensor]] | None = None) -> Tensor:
        if ids is not None and ids.data_ptr() != self.ids.data_ptr():
            self.ids.copy_(ids)
        if states is not None:
            dst = [t for st in self.start for t in st.values()]
            src = [st[k] for st, mine in zip(states, self.start) for k in mine]
            torch._foreach_copy_(dst, src)
        self.graph.replay()
        return self.logits

    def check(self) -> None:
        """Raise ``recurrent.GatedScanTimeoutError`` if a replay's fused gate
        kernel timed out waiting for a carry (reads the status word: a sync)."""

        recurrent.check_gated_scan_status(self.status)


def _stack_decode(params: list[dict[str, Tensor]], settings: HermSettings, ids: Tensor,
                  states: list[dict[str, Tensor]], out_states: list[dict[str, Tensor]] | None = None
                  ) -> tuple[Tensor, list[dict[str, Tensor]]]:
    """One decode position ([B, 1] ids) through every layer, the token context
    formed once for all of them (every layer sees the same ids and carries the
    same last token): one kernel per step instead of one per layer. Otherwise
    ``block_window`` layer after layer. ``out_states``: state dicts whose
    buffers receive the next states (all layers' ``last_token`` one buffer)."""

    ids = ids.contiguous()
    token_context = _token_context(ids, None, states[0]["last_token"],
                                   out_states[0]["last_token"] if out_states is not None else None)
    context = None
    next_states = []
    logits = None
    routing: dict = {}  # the hash route, formed by the first layer for all of them
    surprises = _surprise_layers(params, settings, states, token_context[3], token_context[2])
    for layer, (p, state) in enumerate(zip(params, states)):
        last = layer == len(params) - 1
        logits, context, next_state, _ = block_window(p, settings, ids, state, context, with_logits=last,
                                                      token_context=token_context,
                                                      next_norm=None if last else params[layer + 1]["input_norm"],
                                                      out_state=out_states[layer] if out_states is not None else None,
                                                      routing=routing,
                                                      surprise_in=surprises[layer] if surprises else None)
        next_states.append(next_state)
    return logits, next_states


def stack_window(params: list[dict[str, Tensor]], settings: HermSettings, ids: Tensor,
                 states: list[dict[str, Tensor]]) -> tuple[Tensor, list[dict[str, Tensor]]]:
    """One window through every layer; returns the last layer's logits and the
    next states. Decode steps (one position) take ``_stack_decode``."""

    if ids.shape[1] == 1 and ids.device.type == "cuda":
        return _stack_decode(params, settings, ids, states)
    context = None
    next_states = []
    logits = None
    routing: dict = {}  # the hash route, formed by the first layer for all of them
    for layer, (p, state) in enumerate(zip(params, states)):
        last = layer == len(params) - 1
        logits, context, next_state, _ = block_window(p, settings, ids, state, context, with_logits=last,
                                                      next_norm=None if last else params[layer + 1]["input_norm"],
                                                      routing=routing)
        next_states.append(next_state)
    return logits, next_states


def prefill(params: list[dict[str, Tensor]], settings: HermSettings, ids: Tensor,
            states: list[dict[str, Tensor]]) -> tuple[Tensor, list[dict[str, Tensor]]]:
    """forward_parallel (network.py:176-197): windows of ``scan_chunk`` tokens, state carried."""

    pieces = []
    for start in range(0, ids.shape[1], settings.scan_chunk):
        logits, states = stack_window(params, settings, ids[:, start:start + settings.scan_chunk].contiguous(), states)
        pieces.append(logits)
    return torch.cat(pieces, dim=1), states


def decode_step(params: list[dict[str, Tensor]], settings: HermSettings, ids: Tensor,
                states: list[dict[str, Tensor]]) -> tuple[Tensor, list[dict[str, Tensor]]]:
    """One greedy decode step at fixed shapes: ``ids`` ``[B, 1]`` -> the next ids
    ``[B, 1]`` (argmax of the logits with the padding id removed, as
    TokenSampler does for a greedy policy, runtime/fast_decode.py:53-55, 82-84)
    and the next states."""

    logits, states = stack_window(params, settings, ids, states)
    return _greedy_tokens(logits), states


def _greedy_tokens(logits: Tensor, out: Tensor | None = None) -> Tensor:
    """argmax over the vocabulary of the last position's logits with the
    padding id excluded (its score taken as -inf, the first maximum winning,
    as ``torch.argmax`` after masking does), [B, 1] int64, one kernel
    (``koemi_herm_greedy_tokens``)."""

    batch, length, vocab = logits.shape
    if logits.dtype != torch.float32 or logits.stride(2) != 1:
        logits = logits.float().contiguous()
    ids = out if out is not None else torch.empty((batch, 1), device=logits.device, dtype=torch.int64)
    _native.call("koemi_herm_greedy_tokens", _native.ptr(logits[:, -1]), logits.stride(0), batch, vocab,
                 PAD_TOKEN_ID, _native.ptr(ids), _native.stream_of(logits.device))
    return ids


class WindowGraph:
    """``stack_window`` at a fixed (batch, length) replayed from one captured HIP graph.

    The window (every layer, then copies of the next states into static
    buffers, and with ``greedy`` the next ids of a greedy decode step into the
    static ids) is captured once over private copies of ``states``; each
    ``run()`` copies the given ids in (unless greedy), replays, and leaves the
    last layer's logits in ``self.logits`` and the advanced state in
    ``self.states``. Fixed shapes (static rings), no host synchronisation and
    no allocation inside the replay. Two eager windows on throwaway copies
    warm the libraries up before the capture.
    """

    def __init__(self, params: list[dict[str, Tensor]], settings: HermSettings, states: list[dict[str, Tensor]],
                 ids: Tensor, *, greedy: bool = False) -> None:
        self.params = params
        self.settings = settings
        self.greedy = greedy
        self.ids = ids.clone().contiguous()
        gate_status(self.ids.device)
        self.states = [{k: v.clone() for k, v in st.items()} for st in states]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            warm_ids, warm_states = self.ids.clone(), [{k: v.clone() for k, v in st.items()} for st in states]
            for _ in range(2):
                _, warm_states = stack_window(params, settings, warm_ids, warm_states)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self._window()

    def _window(self) -> Tensor:
        logits, next_states = stack_window(self.params, self.settings, self.ids, self.states)
        # every layer's next state into the static buffers: a few multi-tensor
        # copy kernels (one per dtype) rather than one copy per tensor
        groups: dict[torch.dtype, tuple[list[Tensor], list[Tensor]]] = {}
        for state, new in zip(self.states, next_states):
            for key, tensor in state.items():
                dst, src = groups.setdefault(tensor.dtype, ([], []))
                dst.append(tensor)
                src.append(new[key])
        for dst, src in groups.values():
            torch._foreach_copy_(dst, src)
        if self.greedy:
            _greedy_tokens(logits, out=self.ids)
        return logits

    def run(self, ids: Tensor | None = None) -> Tensor:
        if ids is not None:
            self.ids.copy_(ids)
        self.graph.replay()
        return self.logits


class DecodeGraph:
    """Greedy decode steps (``decode_step``) replayed from two captured HIP
    graphs over two static state sets: step n reads set n % 2 and its kernels
    write the next state straight into set (n + 1) % 2 (``out_state``), so no
    state is copied between steps (the rings alone are 4 x 4 MiB per layer at
    the C5 batch). ``step()`` advances ``self.ids`` ``[B, 1]`` in place and
    ``self.states`` to the new set; ``run()`` does the same and returns the
    step's logits. Every layer of a set shares one ``last_token`` buffer (the
    stack's layers carry the same last token). Two eager steps on throwaway
    copies warm the libraries up before the captures. The next ids are the
    greedy pick, or with a non-greedy ``policy`` (``sampling.SamplingPolicy``)
    TokenSampler's draw (fast_decode.py:76-95) from uniforms that ``run()``
    draws from ``generator`` into a static buffer before each replay. The
    expert weights of ``params`` are given their fragment-order copies first
    (``add_decode_fragments``, in place)."""

    def __init__(self, params: list[dict[str, Tensor]], settings: HermSettings, ids: Tensor,
                 states: list[dict[str, Tensor]], *, policy=None, generator: torch.Generator | None = None) -> None:
        add_decode_fragments(params)
        self.params, self.settings = params, settings
        self.ids = ids.clone().contiguous()
        gate_status(self.ids.device)
        # non-greedy sampling.SamplingPolicy: the captured step draws from
        # self.uniforms, refilled from `generator` before every replay
        self.policy = policy if policy is not None and not policy.greedy else None
        self.generator = generator
        self.uniforms = torch.zeros((self.ids.shape[0],), device=self.ids.device, dtype=torch.float32)
        self._sets = []
        for _ in range(2):
            copy = [{k: v.clone() for k, v in st.items()} for st in states]
            for st in copy[1:]:
                st["last_token"] = copy[0]["last_token"]
            self._sets.append(copy)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            warm_ids, warm_states = self.ids.clone(), [{k: v.clone() for k, v in st.items()} for st in states]
            for _ in range(2):
                _, warm_states = stack_window(params, settings, warm_ids, warm_states)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self._graphs, self._logits = [], []
        for parity in (0, 1):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._logits.append(self._step(self._sets[parity], self._sets[1 - parity]))
            self._graphs.append(graph)
        self._parity = 0

    def _step(self, src: list[dict[str, Tensor]], dst: list[dict[str, Tensor]]) -> Tensor:
        logits, _ = _stack_decode(self.params, self.settings, self.ids, src, dst)
        if self.policy is None:
            _greedy_tokens(logits, out=self.ids)
        else:
            last = logits[:, -1]
            _native.call("koemi_herm_sample_tokens", _native.ptr(last), logits.stride(0), last.shape[0],
                         last.shape[1], PAD_TOKEN_ID, float(self.policy.temperature), int(self.policy.top_k or 0),
                         _native.ptr(self.uniforms), _native.ptr(self.ids), None, _native.stream_of(logits.device))
        return logits

    @property
    def states(self) -> list[dict[str, Tensor]]:
        return self._sets[self._parity]

    @property
    def logits(self) -> Tensor:
        return self._logits[1 - self._parity]

    def run(self) -> Tensor:
        if self.policy is not None:
            self.uniforms.uniform_(0.0, 1.0, generator=self.generator)
        self._graphs[self._parity].replay()
        self._parity ^= 1
        return self.logits

    def step(self) -> Tensor:
        self.run()
        return self.ids


def prefill_graphed(params: list[dict[str, Tensor]], settings: HermSettings, ids: Tensor,
                    states: list[dict[str, Tensor]], graph: WindowGraph | None = None
                    ) -> tuple[Tensor, list[dict[str, Tensor]], WindowGraph]:
    """``prefill`` with every window replayed from one ``WindowGraph`` (the
    sequence length a multiple of ``scan_chunk``). Pass the graph of an earlier
    call to reuse it; its state buffers are reset to ``states`` first."""

    batch, length = ids.shape
    chunk = settings.scan_chunk
    if length % chunk:
        raise ValueError("prefill_graphed needs a length that is a multiple of scan_chunk")
    if graph is None:
        graph = WindowGraph(params, settings, states, ids[:, :chunk])
    for state, start in zip(graph.states, states):
        for key, tensor in state.items():
            tensor.copy_(start[key])
    pieces = []
    for begin in range(0, length, chunk):
        pieces.append(graph.run(ids[:, begin:begin + chunk]).clone())
    return torch.cat(pieces, dim=1), graph.states, graph


class WavefrontPrefill:
    """``prefill`` of the whole stack with the layer windows scheduled as a wavefront.

    Window ``w`` of layer ``l`` needs only window ``w - 1`` of the same layer
    (the carried state) and window ``w`` of layer ``l - 1`` (its final
    context), so every (layer, window) pair on an anti-diagonal ``l + w = d``
    is independent of the others. Each layer runs on its own stream of default
    priority; window ``w`` of layer ``l`` waits (HIP events) for window ``w`` of
    layer ``l - 1`` and, before overwriting its output buffer, for window
    ``w - 2`` of layer ``l + 1``, which read it. Small latency-bound kernels of
    different layers then overlap on the GPU instead of running one after the
    other, and the results are those of ``prefill`` bit for bit (the same
    kernels on the same inputs).

    Each layer's window is captured twice (output buffers alternate by window
    parity) into HIP graphs with static inputs: the window's ids (copied in on
    the layer's stream), the previous layer's output of the same parity, and
    the layer's state, which every replay advances in place. ``run(ids)``
    resets the state to ``states`` (as given at construction, or the
    ``states`` argument) and returns the last layer's logits of every window;
    ``self.states`` holds the final states. Fixed (batch, scan_chunk) shapes;
    the sequence length must be a multiple of ``scan_chunk``.
    """

    def __init__(self, params: list[dict[str, Tensor]], settings: HermSettings, states: list[dict[str, Tensor]],
                 batch: int, device: torch.device) -> None:
        self.params, self.settings = params, settings
        self.layers = len(params)
        gate_status(device)
        chunk = settings.scan_chunk
        self.start = [{k: v.clone() for k, v in st.items()} for st in states]
        self.states = [{k: v.clone() for k, v in st.items()} for st in states]
        self.streams = [torch.cuda.Stream(device) for _ in range(self.layers)]
        self.ids_in = [[torch.zeros((batch, chunk), dtype=torch.int64, device=device) for _ in range(2)]
                       for _ in range(self.layers)]
        # warm the libraries up outside the capture: one eager window on throwaway states
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            warm = [{k: v.clone() for k, v in st.items()} for st in states]
            for _ in range(2):
                _, warm = stack_window(params, settings, self.ids_in[0][0], warm)
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize(device)
        self.graphs: list[list[torch.cuda.CUDAGraph]] = []
        self.out: list[list[Tensor]] = []
        self.logits: list[Tensor | None] = [None, None]
        for layer in range(self.layers):
            graphs, outs = [], []
            for parity in range(2):
                g = torch.cuda.CUDAGraph()
                context = self.out[layer - 1][parity] if layer else None
                last = layer == self.layers - 1
                with torch.cuda.graph(g):
                    logits, final, nxt, _ = block_window(params[layer], settings, self.ids_in[layer][parity],
                                                         self.states[layer], context, with_logits=last)
                    keys = list(self.states[layer])
                    torch._foreach_copy_([self.states[layer][k] for k in keys], [nxt[k] for k in keys])
                graphs.append(g)
                outs.append(final)
                if last:
                    self.logits[parity] = logits
            self.graphs.append(graphs)
            self.out.append(outs)
        torch.cuda.synchronize(device)

    def run(self, ids: Tensor, states: list[dict[str, Tensor]] | None = None) -> Tensor:
        batch, length = ids.shape
        chunk = self.settings.scan_chunk
        if length % chunk or batch != self.ids_in[0][0].shape[0]:
            raise ValueError("WavefrontPrefill.run needs the captured batch and a length that is a multiple of "
                             "scan_chunk")
        windows = length // chunk
        current = torch.cuda.current_stream(ids.device)
        source = self.start if states is None else states
        for state, start in zip(self.states, source):
            for key, tensor in state.items():
                tensor.copy_(start[key])
        vocab = self.logits[0].shape[-1]
        logits = torch.empty((batch, length, vocab), device=ids.device, dtype=self.logits[0].dtype)
        ready = current.record_event()
        for stream in self.streams:
            stream.wait_event(ready)
        done: list[list[torch.cuda.Event | None]] = [[None] * windows for _ in range(self.layers)]
        last = self.layers - 1
        for diagonal in range(windows + self.layers - 1):
            for layer in range(self.layers):
                w = diagonal - layer
                if not 0 <= w < windows:
                    continue
                stream, parity = self.streams[layer], w % 2
                with torch.cuda.stream(stream):
                    if layer:
                        stream.wait_event(done[layer - 1][w])
                    if layer < last and w >= 2:
                        stream.wait_event(done[layer + 1][w - 2])  # the reader of this parity's output
                    self.ids_in[layer][parity].copy_(ids[:, w * chunk:(w + 1) * chunk])
                    self.graphs[layer][parity].replay()
                    if layer == last:
                        logits[:, w * chunk:(w + 1) * chunk].copy_(self.logits[parity])
                    done[layer][w] = stream.record_event()
        for stream in self.streams:
            current.wait_stream(stream)
        logits.record_stream(self.streams[last])
        return logits
