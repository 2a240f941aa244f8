"""MI355X (gfx950) HERM hot path behind Koemi-5HOM's operator fronts.

Module map (reference front -> this package):

* ``koemi.cuda_kernels.dense``  -> ``koemi_amd.dense``     (dense_affine_scan)
* ``koemi.model.cuda_scan``     -> ``koemi_amd.cuda_scan`` (cuda_affine_scan)
* ``koemi.cuda_kernels.core``   -> ``koemi_amd.core``      (fused_rmsnorm_silu)
* ``koemi.cuda_kernels.think``  -> ``koemi_amd.think``     (causal_surprise, ...)
* ``koemi.model.memory`` (LocalKeyValueMemory.read_salient_window, salient_tail, read_window) -> ``koemi_amd.memory``
* ``koemi.model.memory`` (BoundedRecurrentState.gates, + network.py:306-310 scan) -> ``koemi_amd.recurrent``
* ``koemi.cuda_kernels.moe``    -> ``koemi_amd.moe``       (route/permute/grouped MLP/combine)
* ``koemi.cuda_kernels.loader`` -> ``koemi_amd.loader``

Every operator runs from ``libkoemi_hip.so`` (C ABI in ``include/koemi_hip.h``):
hand-written HIP kernels, with rocBLAS for the plain GEMMs of the salient read
and the recurrent gates; none falls back to CPU or to PyTorch.
"""

from koemi_amd.core import fused_rmsnorm_silu, load_core_extension
from koemi_amd.cuda_scan import cuda_affine_scan, diagnose_cuda_affine_scan
from koemi_amd.dense import dense_affine_scan, native_cuda_available
from koemi_amd.memory import read_local_window, read_salient_window, salient_tail
from koemi_amd.recurrent import recurrent_gates, recurrent_scan
from koemi_amd.moe import (
    combine_topk,
    expert_activation_counts,
    grouped_expert_mlp_inference,
    load_native_extension,
    permute_topk,
    route_topk_learned,
    route_topk_modulo,
    route_topk_valid,
)
from koemi_amd.think import benchmark_causal_surprise, causal_surprise, salience_admission, surprise_from_logits

__all__ = [
    "benchmark_causal_surprise",
    "causal_surprise",
    "combine_topk",
    "cuda_affine_scan",
    "dense_affine_scan",
    "diagnose_cuda_affine_scan",
    "expert_activation_counts",
    "fused_rmsnorm_silu",
    "grouped_expert_mlp_inference",
    "load_core_extension",
    "load_native_extension",
    "native_cuda_available",
    "permute_topk",
    "route_topk_learned",
    "route_topk_modulo",
    "route_topk_valid",
    "salience_admission",
    "read_local_window",
    "read_salient_window",
    "recurrent_gates",
    "recurrent_scan",
    "salient_tail",
    "surprise_from_logits",
]
